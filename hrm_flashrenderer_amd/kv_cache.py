"""Paged K/V cache over one shared page pool with a block table.

Counterpart of the reference's caller-side cache, engine/llama_tp.py:21-107
(`PagedKVCache`). The reference keeps a private page array per sequence,
`[B, Hk, P, PS, D]`, grows every sequence to the next power of two of pages
by reallocating and copying the whole cache (llama_tp.py:47-57), and reads
positions and lengths back from the device with `.item()` on every append
(llama_tp.py:69, 89-97).

Here all sequences share one pool `[1, Hk, pool_pages, PS, D]` (the
reference's 5-D layout with a single pool row, so the kernels' page map
applies unchanged) and a block table `[B, max_blocks]` of int32 physical page
ids on the device:

* pages are taken from a host-side free list only when a sequence's length
  crosses a page boundary, and returned by `free(b)` / `reset()`;
* the pool doubles (one device copy) only when the free list runs dry, and
  the block table widens only when a sequence outgrows it;
* lengths are tracked on the host for allocation, and the device `seqlen`
  is advanced by device ops in stream order (an append at the current
  lengths passes `seqlen` itself as the kernel's start positions), so an
  append whose positions are known on the host (`positions=None`, a Python
  int, or a CPU tensor) never waits on the device; a device tensor of
  positions costs one read-back, as in the reference;
* block-table changes are written with a small scatter of the new entries.

The operators consume the cache through `get()` / `block_table`, or directly
through `attention()`.

`layout="per_sequence"` keeps the reference's own layout instead: one page
array per sequence, `k_pages` `[bsz, Hk, P, PS, D]`, with no block table (the
kernels' identity page map). `get()` then feeds the reference's unchanged
caller (engine/llama_tp.py:186-200), which passes no block table. All
sequences grow together by doubling P with one copy, as the reference does
with its power-of-two growth (llama_tp.py:47-57). Appends and lengths work
the same way in both layouts.

`append(..., positions=[B, T])` takes any positions per row, which is the
reference's general path (llama_tp.py:80-99). Consecutive rows are one
append launch. Other rows are one scatter launch (`paged_kv_scatter`) instead
of the reference's per-row Python copies.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from .ops import flash_attn_paged, flash_attn_paged_append, paged_kv_append, paged_kv_scatter

PositionsLike = Union[None, int, torch.Tensor]


class PagedKVCache:
    """Shared-pool paged K/V cache (see the module docstring).

    Arguments follow the reference constructor (engine/llama_tp.py:24-33):
    `init_pages` is the initial number of pages per sequence, so the pool
    starts with `bsz * init_pages` pages. `max_seq_len` (optional) sizes the
    block table (or, per sequence, the pages) up front; it grows on demand
    otherwise. `layout` is "pool" (one shared pool with a block table) or
    "per_sequence" (the reference's `[bsz, Hk, P, PS, D]`, no block table).
    """

    def __init__(self, bsz: int, kv_heads: int, head_dim: int, page_size: int = 128,
                 init_pages: int = 4, device: Union[str, torch.device] = "cuda",
                 dtype: torch.dtype = torch.float16, *, max_seq_len: Optional[int] = None,
                 pool_pages: Optional[int] = None, layout: str = "pool"):
        self.bsz = int(bsz)
        self.kv_heads = int(kv_heads)
        self.head_dim = int(head_dim)
        self.page_size = int(page_size)
        self.device = torch.device(device)
        self.dtype = dtype
        if self.bsz <= 0 or self.kv_heads <= 0 or self.head_dim <= 0 or self.page_size <= 0:
            raise ValueError("bsz, kv_heads, head_dim and page_size must be positive")
        if layout not in ("pool", "per_sequence"):
            raise ValueError('layout must be "pool" or "per_sequence"')
        self.layout = layout
        self._pages_of = [0] * self.bsz       # mapped logical pages per sequence
        self.lengths = [0] * self.bsz         # host copy of seqlen
        self.seqlen = torch.zeros(self.bsz, dtype=torch.int32, device=self.device)
        self.cur_len = 0                      # max length, as the reference tracks it
        if layout == "per_sequence":
            per_seq = max(1, int(init_pages))
            if max_seq_len is not None:
                per_seq = max(per_seq, -(-int(max_seq_len) // self.page_size))
            self.k_pages = torch.empty(self.bsz, self.kv_heads, per_seq, self.page_size,
                                       self.head_dim, device=self.device, dtype=dtype)
            self.v_pages = torch.empty_like(self.k_pages)
            self._bt_host = None
            self._block_table = None
            self._free: List[int] = []
            return
        npages = int(pool_pages) if pool_pages is not None else self.bsz * max(1, int(init_pages))
        npages = max(1, npages)
        self.k_pages = torch.empty(1, self.kv_heads, npages, self.page_size, self.head_dim,
                                   device=self.device, dtype=dtype)
        self.v_pages = torch.empty_like(self.k_pages)
        blocks = max(1, int(init_pages))
        if max_seq_len is not None:
            blocks = max(blocks, -(-int(max_seq_len) // self.page_size))
        self._bt_host = np.full((self.bsz, blocks), -1, dtype=np.int32)
        self._block_table = torch.full((self.bsz, blocks), -1, dtype=torch.int32,
                                       device=self.device)
        self._free: List[int] = list(range(npages - 1, -1, -1))  # pop() yields low ids first

    # ------------------------------------------------------------ queries --
    @property
    def pool_pages(self) -> int:
        """Physical (page, all KV heads) slots held on the device."""
        return int(self.k_pages.size(0) * self.k_pages.size(2))

    @property
    def max_blocks(self) -> int:
        """Logical pages a sequence can hold without growing the cache."""
        if self._bt_host is None:
            return int(self.k_pages.size(2))
        return int(self._bt_host.shape[1])

    @property
    def block_table(self) -> Optional[torch.Tensor]:
        """int32 [bsz, max_blocks] page map of the pool layout (None per sequence)."""
        return self._block_table

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def get(self) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(k_pages, v_pages, seqlen) as in the reference (llama_tp.py:101-102).
        With the pool layout the operators also need
        `block_table=cache.block_table`; without it they raise "B mismatch"
        with that hint. With layout="per_sequence" the reference's call
        (llama_tp.py:187-200, no block table) works as it stands."""
        return self.k_pages, self.v_pages, self.seqlen

    # --------------------------------------------------------- allocation --
    def reserve(self, b: int, end: int) -> None:
        """Map the pages that hold positions [0, end) of sequence b."""
        need = -(-int(end) // self.page_size)
        have = self._pages_of[b]
        if need <= have:
            return
        self._reserve_many([(b, need)])

    def _reserve_many(self, wants: Sequence[Tuple[int, int]]) -> None:
        if self._bt_host is None:
            need = max((n for _, n in wants), default=0)
            if need > self.k_pages.size(2):
                self._grow_per_sequence(max(need, 2 * int(self.k_pages.size(2))))
            for b, n in wants:
                self._pages_of[b] = max(self._pages_of[b], n)
            return
        new_entries = []
        for b, need in wants:
            have = self._pages_of[b]
            if need <= have:
                continue
            if need > self.max_blocks:
                self._widen_table(max(need, 2 * self.max_blocks))
            missing = need - have
            if missing > len(self._free):
                self._grow_pool(missing - len(self._free))
            for p in range(have, need):
                phi = self._free.pop()
                self._bt_host[b, p] = phi
                new_entries.append((b, p, phi))
            self._pages_of[b] = need
        if new_entries:
            idx = torch.tensor(new_entries, dtype=torch.int64)
            vals = idx[:, 2].to(torch.int32)
            rows = idx[:, 0].to(self.device, non_blocking=True)
            cols = idx[:, 1].to(self.device, non_blocking=True)
            self._block_table[rows, cols] = vals.to(self.device, non_blocking=True)

    def _widen_table(self, blocks: int) -> None:
        old = self._bt_host
        host = np.full((self.bsz, blocks), -1, dtype=np.int32)
        host[:, :old.shape[1]] = old
        self._bt_host = host
        dev = torch.full((self.bsz, blocks), -1, dtype=torch.int32, device=self.device)
        dev[:, :old.shape[1]] = self._block_table
        self._block_table = dev

    def _grow_per_sequence(self, pages: int) -> None:
        old = int(self.k_pages.size(2))
        k = torch.empty(self.bsz, self.kv_heads, pages, self.page_size, self.head_dim,
                        device=self.device, dtype=self.dtype)
        v = torch.empty_like(k)
        k[:, :, :old] = self.k_pages
        v[:, :, :old] = self.v_pages
        self.k_pages, self.v_pages = k, v

    def _grow_pool(self, at_least: int) -> None:
        old = self.pool_pages
        new = max(2 * old, old + int(at_least))
        k = torch.empty(1, self.kv_heads, new, self.page_size, self.head_dim,
                        device=self.device, dtype=self.dtype)
        v = torch.empty_like(k)
        k[:, :, :old] = self.k_pages
        v[:, :, :old] = self.v_pages
        self.k_pages, self.v_pages = k, v
        # new ids go to the bottom of the stack so that freed low ids are reused first
        self._free = list(range(new - 1, old - 1, -1)) + self._free

    def free(self, b: int) -> None:
        """Release sequence b's pages and set its length to zero."""
        n = self._pages_of[b]
        if n and self._bt_host is None:
            self._pages_of[b] = 0   # per-sequence pages stay allocated
        elif n:
            ids = self._bt_host[b, :n].tolist()
            self._free.extend(reversed(ids))
            self._bt_host[b, :n] = -1
            self._block_table[b, :n] = -1
            self._pages_of[b] = 0
        self._set_lengths({b: 0}, shrink=True)

    def reset(self) -> None:
        """Forget every sequence but keep the pool (llama_tp.py:104-107)."""
        for b in range(self.bsz):
            self.free(b)
        self.cur_len = 0

    # ------------------------------------------------------------- append --
    def _starts(self, positions: PositionsLike, T: int) -> Union[List[int], torch.Tensor]:
        """Per-sequence start positions of consecutive rows, or the host
        int64 [B, T] positions when some row is not consecutive."""
        if positions is None:
            return list(self.lengths)
        if isinstance(positions, int):
            return [int(positions)] * self.bsz
        if not isinstance(positions, torch.Tensor):
            positions = torch.as_tensor(positions)
        pos = positions.detach()
        if pos.device.type != "cpu":
            pos = pos.cpu()  # one read-back, like the reference's .item() calls
        if pos.dim() == 1:
            # the reference's fast path reads positions[0] only and writes the
            # T tokens from there (engine/llama_tp.py:67-74)
            if T and pos.numel() == 0:
                raise ValueError("positions [T] must hold the start position")
            start = int(pos[0]) if T else 0
            return [start] * self.bsz
        if pos.dim() == 2:
            if tuple(pos.shape) != (self.bsz, T):
                raise ValueError("positions [B, T] must match k_new")
            starts = pos[:, 0].tolist() if T else [0] * self.bsz
            want = torch.tensor(starts, dtype=torch.int64)[:, None] + torch.arange(T)[None]
            if T and not torch.equal(pos.to(torch.int64), want):
                return pos.to(torch.int64)   # scattered rows
            return [int(s) for s in starts]
        raise ValueError("positions must be None, an int, [T] or [B, T]")

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor,
               positions: PositionsLike = None, *, rope=None,
               valid: Optional[Sequence[int]] = None) -> None:
        """Write k_new / v_new `[B, Hk, T, D]` at positions start_b .. start_b+T-1.

        `positions`: None (append at each sequence's current length), an int
        or a `[T]` tensor (same start for all sequences, positions[0], as the
        reference's fast path, llama_tp.py:65-78, which reads no other entry),
        or `[B, T]` (any positions per row,
        the reference's general path, llama_tp.py:80-99: a row of
        consecutive positions is appended from its start, other rows are
        scattered token by token; of two tokens of one row at the same
        position the later one is kept, as in the reference's loop). One
        kernel launch in every case. `rope=(cos, sin)` rotates each key at
        its own position in the same launch (the reference's apply_rope on
        K, engine/llama_tp.py:183).

        Lengths: each sequence's becomes max(its length, start + T). The
        reference's fast path instead sets every sequence's length to the
        largest end so far (cur_len, llama_tp.py:76-77). The two agree while
        the sequences have equal lengths, which is all the reference's caller
        produces. After ragged appends, the reference's rule would make a
        short sequence attend slots nothing wrote; here each sequence keeps
        its own length.

        `valid` (host ints, one per sequence, each <= T): only the first
        valid[b] tokens of sequence b are real (a ragged chunk padded to T);
        its length becomes max(length, start_b + valid[b]) when valid[b] > 0
        and stays put when it is 0. Pages are mapped for the real tokens only;
        a padding token lands beyond the length in one of the sequence's own
        pages or is skipped by the kernel (unmapped page). Padding must not
        cover live tokens: a sequence whose length exceeds start_b + valid[b]
        with valid[b] < T is rejected.
        """
        B, Hk, T, D = k_new.shape
        if B != self.bsz or Hk != self.kv_heads or D != self.head_dim:
            raise ValueError("k_new must be [bsz, kv_heads, T, head_dim]")
        starts = self._starts(positions, T)
        if isinstance(starts, torch.Tensor):
            if valid is not None:
                raise ValueError("valid applies to rows of consecutive positions only")
            self._scatter(k_new, v_new, starts, rope)
            return
        if any(s < 0 for s in starts):
            raise ValueError("positions must be non-negative")
        if valid is not None:
            valid = [int(x) for x in valid]
            if len(valid) != B or any(x < 0 or x > T for x in valid):
                raise ValueError("valid must hold B counts in [0, T]")
            for b, (st, n) in enumerate(zip(starts, valid)):
                if n < T and self.lengths[b] > st + n:
                    raise ValueError(f"padding tokens of sequence {b} would overwrite "
                                     f"positions below its length {self.lengths[b]}")
        if T == 0:
            return
        counts = valid if valid is not None else [T] * B
        self._reserve_many([(b, -(-(s + n) // self.page_size)) for b, (s, n)
                            in enumerate(zip(starts, counts)) if n > 0])
        uniform = len(set(starts)) == 1
        if uniform:
            start_arg: Union[int, torch.Tensor] = starts[0]
        elif positions is None:
            start_arg = self.seqlen  # the current lengths, already on the device
        else:
            start_arg = torch.tensor(starts, dtype=torch.int32).to(self.device, non_blocking=True)
        paged_kv_append(self.k_pages, self.v_pages, k_new.contiguous(), v_new.contiguous(),
                        start_arg, self.page_size, block_table=self._block_table, rope=rope)
        # seqlen = max(seqlen, start + count), in stream order after the kernel
        if valid is not None:
            ends = [st + n if n > 0 else 0 for st, n in zip(starts, counts)]
            ends_dev = torch.tensor(ends, dtype=torch.int32).to(self.device, non_blocking=True)
            torch.maximum(self.seqlen, ends_dev, out=self.seqlen)
        elif uniform:
            self.seqlen.clamp_(min=starts[0] + T)
        elif positions is None:
            self.seqlen.add_(T)
        else:
            torch.maximum(self.seqlen, start_arg + T, out=self.seqlen)
        for b, (st, n) in enumerate(zip(starts, counts)):
            if n > 0:
                self.lengths[b] = max(self.lengths[b], st + n)
        self.cur_len = max(self.lengths)

    def _scatter(self, k_new: torch.Tensor, v_new: torch.Tensor, pos: torch.Tensor, rope) -> None:
        """Token t of sequence b at pos[b, t] (host int64 [B, T]), one launch."""
        if bool((pos < 0).any()):
            raise ValueError("positions must be non-negative")
        ends = (pos.max(dim=1).values + 1).tolist()
        self._reserve_many([(b, -(-int(e) // self.page_size)) for b, e in enumerate(ends)])
        keep = keep_last_of_duplicates(pos.numpy())
        pos_dev = torch.from_numpy(keep.astype(np.int32)).to(self.device, non_blocking=True)
        paged_kv_scatter(self.k_pages, self.v_pages, k_new.contiguous(), v_new.contiguous(),
                         pos_dev, self.page_size, block_table=self._block_table, rope=rope)
        ends_dev = torch.tensor(ends, dtype=torch.int32).to(self.device, non_blocking=True)
        torch.maximum(self.seqlen, ends_dev, out=self.seqlen)
        for b, e in enumerate(ends):
            self.lengths[b] = max(self.lengths[b], int(e))
        self.cur_len = max(self.lengths)

    def _set_lengths(self, new: dict, shrink: bool = False) -> None:
        for b, n in new.items():
            if shrink or n > self.lengths[b]:
                self.lengths[b] = int(n)
                self.seqlen[b].fill_(int(n))
        self.cur_len = max(self.lengths) if self.lengths else 0

    # ---------------------------------------------------------- attention --
    def attention(self, q: torch.Tensor, head_map: torch.Tensor, causal: bool,
                  q_offset: Union[int, torch.Tensor] = 0, *, rope=None,
                  q_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
        """flash_attn_paged over this cache (block table included); `rope`
        rotates q in the kernel at positions q_offset + i; `q_lens` (int32
        [B] on the device) marks rows i >= q_lens[b] as padding (zeros)."""
        return flash_attn_paged(q, self.k_pages, self.v_pages, self.seqlen, self.page_size,
                                head_map, causal, q_offset, 0, block_table=self._block_table,
                                rope=rope, q_lens=q_lens)

    def decode_step(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                    head_map: torch.Tensor, *, causal: bool = False, rope=None) -> torch.Tensor:
        """One decode step in one call: append k_new / v_new `[B, Hk, 1, D]` at
        every sequence's current length and attend with q `[B, Hq, M, D]`
        over the lengths that include the new token.

        The same as `append(k_new, v_new)` then `attention(q, head_map,
        causal, q_offset=lengths, rope=rope)` (the reference's decode step,
        engine/llama_tp.py:183-200), but the lengths advance on the device and,
        without rope, the append needs no launch of its own when the attention
        runs on the decode kernels (see flash_attn_paged_append). The query rows sit at
        the new token's position (q_offset = the lengths before the step).
        """
        B, Hk, T, D = k_new.shape
        if B != self.bsz or Hk != self.kv_heads or D != self.head_dim or T != 1:
            raise ValueError("k_new must be [bsz, kv_heads, 1, head_dim]")
        self._reserve_many([(b, -(-(n + 1) // self.page_size)) for b, n in enumerate(self.lengths)])
        o = flash_attn_paged_append(q, self.k_pages, self.v_pages, k_new.contiguous(),
                                    v_new.contiguous(), self.seqlen, self.page_size, head_map,
                                    causal, block_table=self._block_table, rope=rope)
        self.lengths = [n + 1 for n in self.lengths]
        self.cur_len = max(self.lengths)
        return o

    def prefill_chunk(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                      starts: Sequence[int], valid: Sequence[int], head_map: torch.Tensor,
                      *, rope=None) -> torch.Tensor:
        """One chunk of a chunked prefill in which every sequence has its own
        position (a `chunked_prefill_schedule` entry).

        Row i < valid[b] of sequence b is the prompt token at position
        starts[b] + i; rows past valid[b] are padding. The chunk's K/V are
        appended at those positions (padding maps no page and never covers a
        live token), then the chunk attends causally over each sequence's
        cache with q_offset = starts (int32 [B]) and q_lens = valid, so the
        kernels skip the padding rows' tiles and return zeros for them.
        Returns the attention output [B, Hq, T, D]. This generalises the
        reference's generate loop (engine/llama_tp.py:338-354), which runs
        equal-length prompts at one shared position.
        """
        B, _, T, _ = k_new.shape
        starts = [int(x) for x in starts]
        valid = [int(x) for x in valid]
        if len(starts) != B or len(valid) != B:
            raise ValueError("starts and valid must hold B entries")
        pos = torch.tensor(starts, dtype=torch.int64)[:, None] + torch.arange(T)[None]
        self.append(k_new, v_new, pos, valid=valid, rope=rope)
        qo = torch.tensor(starts, dtype=torch.int32).to(self.device, non_blocking=True)
        ql = torch.tensor(valid, dtype=torch.int32).to(self.device, non_blocking=True)
        return self.attention(q, head_map, True, qo, rope=rope, q_lens=ql)


def chunked_prefill_schedule(prompt_lengths: Sequence[int], chunk_tokens: int,
                             cached_lengths: Optional[Sequence[int]] = None
                             ) -> List[Tuple[List[int], List[int]]]:
    """Chunks of a chunked prefill in which each sequence advances from its
    own position.

    Sequence b already holds cached_lengths[b] tokens (0 by default; a shared
    prefix or an earlier turn) and has prompt_lengths[b] new tokens. Chunk c
    takes new tokens [c * chunk_tokens, (c + 1) * chunk_tokens) of every
    sequence, at positions cached_lengths[b] + c * chunk_tokens + i. Returns
    [(starts, valid), ...]: starts[b] is the chunk's first position in
    sequence b (its q_offset), valid[b] how many of its rows are real (its
    q_lens; 0 once the sequence's prompt is done). A chunk's row count is
    max(valid). Feed each entry to `PagedKVCache.prefill_chunk`. With equal
    prompts and no cache this is the reference's loop (engine/llama_tp.py:
    338-354); ragged prompts and prefixes need no padding work, because the
    kernels skip rows past valid[b].
    """
    if chunk_tokens <= 0:
        raise ValueError("chunk_tokens must be positive")
    n = [int(x) for x in prompt_lengths]
    cached = [0] * len(n) if cached_lengths is None else [int(x) for x in cached_lengths]
    if len(cached) != len(n):
        raise ValueError("cached_lengths must match prompt_lengths")
    if any(x < 0 for x in n) or any(x < 0 for x in cached):
        raise ValueError("lengths must be non-negative")
    plan = []
    for c in range(0, max(n, default=0), chunk_tokens):
        valid = [max(0, min(chunk_tokens, x - c)) for x in n]
        plan.append(([cb + c for cb in cached], valid))
    return plan


def keep_last_of_duplicates(pos: np.ndarray) -> np.ndarray:
    """Copy of `pos` [B, T] in which every position that occurs again later
    in its row is replaced by -1 (a slot the scatter kernel skips), so the
    last token written to a position wins, as in the reference's loop over t
    (engine/llama_tp.py:92-97)."""
    keep = np.array(pos, dtype=np.int64, copy=True)
    T = keep.shape[1] if keep.ndim == 2 else 0
    for row in keep:
        _, last_rev = np.unique(row[::-1], return_index=True)
        drop = np.ones(T, dtype=bool)
        drop[T - 1 - last_rev] = False
        row[drop] = -1
    return keep


def chunked_prefill_plan(prompt_lengths: Sequence[int], chunk_tokens: int) -> List[Tuple[int, List[int]]]:
    """Chunks of a chunked prefill over prompts of different lengths.

    The reference's generate loop (engine/llama_tp.py:339-354) prefills a batch
    of equal-length prompts in chunks of `prefill_chunk_size` tokens at one
    shared position. With ragged prompts, chunk c still starts every sequence
    at position c * chunk_tokens (a scalar q_offset), and `valid[b]` says how
    many of its tokens belong to prompt b. Pass it to `PagedKVCache.append`;
    rows beyond `valid[b]` of the chunk's attention output are padding.
    Returns [(start, valid), ...] for as many chunks as the longest prompt needs.
    """
    if chunk_tokens <= 0:
        raise ValueError("chunk_tokens must be positive")
    longest = max((int(n) for n in prompt_lengths), default=0)
    plan = []
    for start in range(0, longest, chunk_tokens):
        plan.append((start, [max(0, min(chunk_tokens, int(n) - start)) for n in prompt_lengths]))
    return plan
