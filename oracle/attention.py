"""CPU oracle of the attention path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker (or, for the baseline, as the timed CPU
restatement). The product path (hrm_flashrenderer_amd) never imports it.

Contents
  1. fp64 closed form (numpy): the tolerance target of every GPU parity test
     (outputs within 2e-3 + 1e-2*|ref| of the exact softmax attention).
       attention_f64            O = softmax(Q K^T / sqrt(D) + mask) V
       decode_token_major_f64   the INT8 engine's decode step over its
                                token-major cache (deepseek_native_engine.sh:562-604)
  2. Page-map helpers (numpy): the reference's paged layout and the additive
     block-table indirection; the rotary embedding the fused kernels apply.
       gather_kv                pages -> contiguous [B, Hk, cap, D]
       append_f16               closed-form index map of paged_kv_append
       rope_tables, rope_f16    engine/rope.py:6-24 (tables; fp16 apply_rope)
  3. Restatement of the reference's CPU math path (torch, same operation
     sequence and dtypes as flashattention_custom/ops.py:19-72), the "port"
     timed as the CPU baseline; pinned bit-for-bit by the golden vectors in
     tests/golden/ that the reference itself produced.
       cpu_flash_attn           ops.py:19-31
       cpu_flash_attn_paged     ops.py:34-60 (+ block table / per-seq offsets)
       cpu_paged_kv_append      ops.py:63-72 (+ block table / per-seq starts)

How each function is pinned (tests/test_oracle.py):
  attention_f64     brute-force triple loop on tiny shapes; torch SDPA in
                    float64 with an explicit mask; invariants (one visible key
                    -> v, equal scores -> mean of V, shift invariance, key
                    permutation invariance, GQA == MHA with repeated K/V).
  decode_token_major_f64
                    == attention_f64 on the re-laid-out cache with head map
                    h % KVH; == a per-key transcription of the engine's online
                    recurrence (m, s, acc) on a tiny case; t = 0 gives v_0; a
                    planted h // group head map fails.
  gather_kv         identity block table == reference flatten (ops.py:43-45);
                    a permuted pool gathered == the unpermuted original.
  append_f16        the reference's append known-answer test shape
                    (flash_tests/test_append_fast.py:16-38) against an
                    independent per-element loop; page-crossing starts.
  rope_f16          bit-exact against torch's own fp16 CPU arithmetic on the
                    same expression; position 0 is the identity; each
                    rotated pair keeps its norm; rotating by p1 then p2
                    matches rotating by p1 + p2; a planted sign error fails.
  rope_tables       against the closed form cos/sin of t * theta^(-j/half)
                    in float64 (to fp16 rounding).
  cpu_*             golden vectors written by the reference's own ops.py.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Union

import numpy as np
import torch

ArrayLike = Union[np.ndarray, torch.Tensor]


def _np(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def _per_seq(v, B: int) -> np.ndarray:
    if isinstance(v, (int, np.integer)):
        return np.full(B, int(v), dtype=np.int64)
    return _np(v).astype(np.int64).reshape(B)


# --------------------------------------------------------------------------
# 1. fp64 closed form
# --------------------------------------------------------------------------

def attention_f64(q: ArrayLike, k: ArrayLike, v: ArrayLike, causal: bool = True,
                  q_offset=0, k_offset=0, kv_len: Optional[Sequence[int]] = None,
                  head_map: Optional[Sequence[int]] = None) -> np.ndarray:
    """Exact softmax attention in float64.

    q [B,Hq,M,D]; k, v [B,Hk,N,D] (contiguous view of the keys of each
    sequence). Key j is visible to row i of sequence b iff j < kv_len[b] and,
    when causal, k_off[b] + j <= q_off[b] + i (reference semantics:
    flash_attn_sm75.cu:65-71, :164, :328; ops.py:25-29, :53-57). q head h reads
    K/V head head_map[h] (default h // (Hq // Hk)).
    A row with no visible key is NaN when kv_len > 0 and 0 when kv_len == 0
    (empty softmax times empty V), matching ops.py.
    """
    qn = _np(q).astype(np.float64)
    kn = _np(k).astype(np.float64)
    vn = _np(v).astype(np.float64)
    B, Hq, M, D = qn.shape
    Hk, N = kn.shape[1], kn.shape[2]
    lens = np.full(B, N, dtype=np.int64) if kv_len is None else _np(kv_len).astype(np.int64)
    lens = np.clip(lens, 0, N)
    qo = _per_seq(q_offset, B)
    ko = _per_seq(k_offset, B)
    hmap = (np.arange(Hq) // (Hq // Hk)) if head_map is None else _np(head_map).astype(np.int64)
    scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, Hq, M, D), dtype=np.float64)
    for b in range(B):
        n = int(lens[b])
        if n == 0:
            continue
        j = np.arange(n)
        i = np.arange(M)
        vis = np.ones((M, n), dtype=bool)
        if causal:
            vis = (ko[b] + j)[None, :] <= (qo[b] + i)[:, None]
        for h in range(Hq):
            hk = int(hmap[h])
            if not (0 <= hk < Hk):
                out[b, h] = np.nan
                continue
            s = (qn[b, h] @ kn[b, hk, :n].T) * scale
            s = np.where(vis, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            with np.errstate(invalid="ignore"):
                e = np.exp(s - mx)
                p = e / e.sum(axis=1, keepdims=True)
            out[b, h] = p @ vn[b, hk, :n]
    return out


def decode_token_major_f64(q: ArrayLike, k_cache: ArrayLike, v_cache: ArrayLike, t: int,
                           scale: Optional[float] = None,
                           head_map: Optional[Sequence[int]] = None) -> np.ndarray:
    """Decode attention of the reference's INT8 engine in float64.

    attn_decode (scripts/deepseek_native_engine.sh:562-604): query head h
    attends keys 0..t of KV head kvh = h % KVH (:568; or head_map[h]) in the
    token-major fp16 cache written by kv_store (:553-559), row j of head kvh at
    j*KVH*Dh + kvh*Dh; scale = 1/sqrt(Dh) as launched (:1077).
    q [H, Dh]; k_cache, v_cache [T, KVH, Dh] with T > t. Returns [H, Dh].
    """
    qn = _np(q).astype(np.float64)
    kn = _np(k_cache).astype(np.float64)
    vn = _np(v_cache).astype(np.float64)
    H, Dh = qn.shape
    KVH = kn.shape[1]
    sc = 1.0 / math.sqrt(Dh) if scale is None else float(scale)
    hmap = np.arange(H) % KVH if head_map is None else _np(head_map).astype(np.int64)
    out = np.zeros((H, Dh), dtype=np.float64)
    for h in range(H):
        kvh = int(hmap[h])
        if not (0 <= kvh < KVH):
            out[h] = np.nan
            continue
        s = (kn[:t + 1, kvh] @ qn[h]) * sc
        e = np.exp(s - s.max())
        out[h] = (e / e.sum()) @ vn[:t + 1, kvh]
    return out


def within_tolerance(out: ArrayLike, ref: ArrayLike, atol: float = 2e-3, rtol: float = 1e-2):
    """Elementwise |out - ref| <= atol + rtol*|ref| (NaN must match NaN).

    Returns (ok, max_excess) where max_excess = max(|out-ref| - rtol*|ref|).
    """
    o = _np(out).astype(np.float64)
    r = _np(ref).astype(np.float64)
    nan_o, nan_r = np.isnan(o), np.isnan(r)
    if not np.array_equal(nan_o, nan_r):
        return False, float("inf")
    mask = ~nan_r
    err = np.abs(o[mask] - r[mask]) - rtol * np.abs(r[mask])
    worst = float(err.max()) if err.size else 0.0
    return worst <= atol, worst


# --------------------------------------------------------------------------
# 2. page maps
# --------------------------------------------------------------------------

def physical_page(b: int, p: int, P: int, block_table: Optional[np.ndarray]) -> int:
    """Physical id of logical page p of sequence b (identity map b*P + p without a table)."""
    if block_table is None:
        return b * P + p
    return int(block_table[b, p])


def gather_kv(pages: ArrayLike, B: int, page_size: int,
              block_table: Optional[ArrayLike] = None) -> np.ndarray:
    """Gather a paged pool [NB,Hk,P,PS,D] into contiguous [B,Hk,cap,D].

    cap = P*PS without a block table (the reference flatten of ops.py:43-45),
    else max_blocks*PS; logical page p of sequence b is pool page
    phi = block_table[b, p] -> pages[phi // P, :, phi % P]. Unmapped pages
    (phi < 0) read as NaN so that any use of them is visible.
    """
    pg = _np(pages)
    NB, Hk, P, PS, D = pg.shape
    assert PS == page_size
    bt = None if block_table is None else _np(block_table).astype(np.int64)
    nblk = P if bt is None else bt.shape[1]
    out = np.full((B, Hk, nblk * PS, D), np.nan, dtype=pg.dtype)
    for b in range(B):
        for p in range(nblk):
            phi = physical_page(b, p, P, bt)
            if phi < 0 or phi >= NB * P:
                continue
            out[b, :, p * PS:(p + 1) * PS] = pg[phi // P, :, phi % P]
    return out


def append_f16(k_pages: ArrayLike, v_pages: ArrayLike, k_new: ArrayLike, v_new: ArrayLike,
               start_pos, page_size: int, block_table: Optional[ArrayLike] = None):
    """Closed-form result of paged_kv_append (returns new numpy arrays).

    pos = start_b + t goes to logical page pos // PS, slot pos % PS
    (flash_attn_sm75.cu:545-554, ops.py:63-72); positions whose page is
    negative, beyond the capacity, or unmapped are skipped (:548).
    """
    kp = _np(k_pages).copy()
    vp = _np(v_pages).copy()
    kn = _np(k_new)
    vn = _np(v_new)
    B, Hk, T, D = kn.shape
    NB, _, P, PS, _ = kp.shape
    assert PS == page_size
    bt = None if block_table is None else _np(block_table).astype(np.int64)
    nblk = P if bt is None else bt.shape[1]
    starts = _per_seq(start_pos, B)
    for b in range(B):
        pos = starts[b] + np.arange(T)
        page = np.floor_divide(pos, PS)
        slot = pos - page * PS
        ok = (pos >= 0) & (page < nblk)
        for t in np.nonzero(ok)[0]:
            phi = physical_page(b, int(page[t]), P, bt)
            if phi < 0 or phi >= NB * P:
                continue
            kp[phi // P, :, phi % P, slot[t]] = kn[b, :, t]
            vp[phi // P, :, phi % P, slot[t]] = vn[b, :, t]
    return kp, vp


def rope_tables(max_len: int, head_dim: int, theta: float = 10000.0):
    """cos/sin fp16 tables [max_len, D/2] as engine/rope.py:6-13 builds them:
    inv_freq_j = theta^(-j/half), angle = t * inv_freq_j in fp32, then cos/sin
    rounded to fp16. Returns numpy float16 arrays."""
    half = head_dim // 2
    inv = 1.0 / (np.float32(theta) ** (np.arange(half, dtype=np.float32) / np.float32(half)))
    ang = np.arange(max_len, dtype=np.float32)[:, None] * inv.astype(np.float32)[None, :]
    return np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)


def rope_f16(x: ArrayLike, cos: ArrayLike, sin: ArrayLike, positions) -> np.ndarray:
    """apply_rope of engine/rope.py:15-24 in its fp16 operation order.

    x [..., T, D] fp16 with the half-split layout x1 = x[..., :D/2],
    x2 = x[..., D/2:]; c = cos[positions], s = sin[positions] ([T, D/2], or
    [..., T, D/2] for per-row positions); y1 = x1*c - x2*s, y2 = x1*s + x2*c,
    where every product and every sum is rounded to fp16 (torch's fp16 ops
    compute in fp32 and round once; fp32 holds the product of two fp16 values
    exactly). Returns float16.
    """
    xv = _np(x).astype(np.float16)
    D = xv.shape[-1]
    half = D // 2
    pos = np.asarray(positions, dtype=np.int64)
    c = _np(cos).astype(np.float16)[pos].astype(np.float32)
    s = _np(sin).astype(np.float16)[pos].astype(np.float32)
    x1 = xv[..., :half].astype(np.float32)
    x2 = xv[..., half:].astype(np.float32)
    r = lambda v: v.astype(np.float16).astype(np.float32)  # noqa: E731
    y1 = (r(x1 * c) - r(x2 * s)).astype(np.float16)
    y2 = (r(x1 * s) + r(x2 * c)).astype(np.float16)
    return np.concatenate([y1, y2], axis=-1)


# --------------------------------------------------------------------------
# 3. restatement of the reference's CPU math path (torch)
# --------------------------------------------------------------------------

def _mask_scores(scores: torch.Tensor, causal: bool, q_off: int, k_off: int) -> torch.Tensor:
    if not causal:
        return scores
    M, N = scores.shape[-2], scores.shape[-1]
    rows = torch.arange(q_off, q_off + M)
    cols = torch.arange(k_off, k_off + N)
    hidden = cols.view(*([1] * (scores.dim() - 1)), N) > rows.view(*([1] * (scores.dim() - 2)), M, 1)
    return scores.masked_fill(hidden, float("-inf"))


def cpu_flash_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
                   q_offset: int = 0, k_offset: int = 0) -> torch.Tensor:
    """ops.py:19-31: fp32 scores and softmax, P cast to q.dtype, batched P @ V."""
    inv_sqrt_d = 1.0 / math.sqrt(q.shape[-1])
    scores = torch.matmul(q.float(), k.float().transpose(-1, -2)) * inv_sqrt_d
    scores = _mask_scores(scores, causal, int(q_offset), int(k_offset))
    probs = torch.softmax(scores, dim=-1).to(q.dtype)
    return torch.matmul(probs, v)


def cpu_flash_attn_paged(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                         seqlen: torch.Tensor, page_size: int, head_map: torch.Tensor,
                         causal: bool = True, q_offset=0, k_offset=0,
                         block_table: Optional[torch.Tensor] = None,
                         batches: Optional[Sequence[int]] = None,
                         heads: Optional[Sequence[int]] = None) -> torch.Tensor:
    """ops.py:34-60: per sequence, flatten its first ceil(slen/PS) pages, then
    per query head a 2-D fp32 score matmul, fp32 softmax cast to q.dtype, and
    P @ V in q.dtype, written into a zero-initialised output.

    Extensions (identity when absent): a block table selects the pool pages of
    each sequence; per-sequence q/k offsets; `batches` / `heads` restrict the
    work to a subset of sequences / query heads (the bounded CPU-baseline
    sample).
    """
    B, Hq, M, D = q.shape
    _, Hk, P, PS, _ = k_pages.shape
    out = torch.zeros_like(q)
    scale = 1.0 / math.sqrt(D)
    qo = _per_seq(q_offset, B) if isinstance(q_offset, torch.Tensor) else None
    ko = _per_seq(k_offset, B) if isinstance(k_offset, torch.Tensor) else None
    for b in (range(B) if batches is None else batches):
        slen = int(seqlen[b].item())
        npages = (slen + page_size - 1) // page_size
        if block_table is None:
            kb = k_pages[b, :, :npages]
            vb = v_pages[b, :, :npages]
        else:
            phys = block_table[b, :npages].long()
            kb = k_pages[phys // P, :, phys % P].transpose(0, 1)
            vb = v_pages[phys // P, :, phys % P].transpose(0, 1)
        k_seq = kb.reshape(Hk, npages * page_size, D)[:, :slen, :]
        v_seq = vb.reshape(Hk, npages * page_size, D)[:, :slen, :]
        q_off = int(qo[b]) if qo is not None else int(q_offset)
        k_off = int(ko[b]) if ko is not None else int(k_offset)
        for h in (range(Hq) if heads is None else heads):
            hk = int(head_map[h].item())
            s = q[b, h].float() @ k_seq[hk].float().t() * scale
            s = _mask_scores(s, causal, q_off, k_off)
            probs = torch.softmax(s, dim=-1).to(q.dtype)
            out[b, h] = probs @ v_seq[hk].to(q.dtype)
    return out


def cpu_paged_kv_append(k_pages: torch.Tensor, v_pages: torch.Tensor, k_new: torch.Tensor,
                        v_new: torch.Tensor, start_pos, page_size: int,
                        block_table: Optional[torch.Tensor] = None) -> None:
    """ops.py:63-72: per sequence and token, copy the [Hk, D] slice into its slot (in place)."""
    B, Hk, T, D = k_new.shape
    P = k_pages.shape[2]
    starts = _per_seq(start_pos, B)
    for b in range(B):
        for t in range(T):
            pos = int(starts[b]) + t
            page, slot = pos // page_size, pos % page_size
            if block_table is None:
                nb, pp = b, page
            else:
                phi = int(block_table[b, page].item())
                nb, pp = phi // P, phi % P
            k_pages[nb, :, pp, slot, :] = k_new[b, :, t, :]
            v_pages[nb, :, pp, slot, :] = v_new[b, :, t, :]
