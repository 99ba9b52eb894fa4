"""Seeded synthetic workloads of the five benchmark configurations, and their
algorithmic cost (flops / bytes) used for roofline fractions.

Configurations (shapes of the reference's target models):
  1  causal MHA prefill, B=1, H=8, S=512, D=64, fp32 and fp16 (contiguous)
  2  causal GQA prefill, Qwen-32B 40/8 heads, D=128, B=4, S=2048, 16-token pages
  3  paged decode, Qwen-32B 40/8, D=128, B=32, context U[512, 8192]
  4  append one token + paged decode, Llama-70B 64/8, D=128, B=64,
     context U[1024, 16384]
  5  chunked prefill, Llama-70B 64/8, D=128, 16 sequences x 512 queries over a
     prior context U[0, 32768]

Paged configurations use one shared pool k_pages/v_pages [1, Hk, NUM_PAGES,
16, 128] and a block table [B, max_blocks] that is a seeded random
permutation of the pool's pages split sequentially over the sequences
(padding entries are -1), i.e. the block-table extension of flash_attn_paged.

Generation order (one CPU generator per config, seed 1000 + config index):
lengths -> block-table permutation; the K/V pool, Q and new K/V are drawn
N(0, 1) in fp32 on the target device from a device generator with the same
seed and cast to fp16.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch

PAGE = 16


@dataclass
class PagedWorkload:
    name: str
    q: torch.Tensor                 # [B, Hq, M, D] fp16
    k_pool: torch.Tensor            # [1, Hk, NUM_PAGES, PS, D] fp16
    v_pool: torch.Tensor
    block_table: torch.Tensor       # int32 [B, max_blocks]
    seqlen: torch.Tensor            # int32 [B]: keys attended (after any append)
    head_map: torch.Tensor          # int32 [Hq]
    causal: bool
    lengths: List[int]              # host copy of seqlen
    q_offsets: Optional[torch.Tensor] = None   # int32 [B] (chunked prefill)
    q_offsets_host: Optional[List[int]] = None
    q_lens: Optional[torch.Tensor] = None      # int32 [B]: live rows of a ragged chunk
    q_lens_host: Optional[List[int]] = None
    k_new: Optional[torch.Tensor] = None       # [B, Hk, 1, D] (decode + append)
    v_new: Optional[torch.Tensor] = None
    append_pos: Optional[torch.Tensor] = None  # int32 [B]
    meta: dict = field(default_factory=dict)

    @property
    def B(self):
        return self.q.size(0)

    @property
    def Hq(self):
        return self.q.size(1)

    @property
    def M(self):
        return self.q.size(2)

    @property
    def D(self):
        return self.q.size(3)

    @property
    def Hk(self):
        return self.k_pool.size(1)


def _device_gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn_f16(shape, gen, device, chunk=1 << 26):
    """N(0,1) fp16 tensor drawn in fp32 chunks (bounded temporary memory)."""
    out = torch.empty(shape, dtype=torch.float16, device=device)
    flat = out.view(-1)
    for s in range(0, flat.numel(), chunk):
        e = min(flat.numel(), s + chunk)
        flat[s:e] = torch.randn(e - s, generator=gen, device=device, dtype=torch.float32).half()
    return out


def _paged(name, cfg_index, B, Hq, Hk, D, M, lengths, causal, device, max_blocks=None,
           q_offsets=None, with_append=False):
    """Pool + block table for sequences of the given lengths (tokens cached)."""
    g = torch.Generator().manual_seed(1000 + cfg_index)
    if lengths is None:
        raise ValueError("lengths required")
    pages = [(n + PAGE - 1) // PAGE for n in lengths]
    total = sum(pages)
    if max_blocks is None:
        max_blocks = max(pages)
    perm = torch.randperm(total, generator=g).to(torch.int32)
    bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    dg = _device_gen(device, 1000 + cfg_index)
    k_pool = _randn_f16((1, Hk, total, PAGE, D), dg, device)
    v_pool = _randn_f16((1, Hk, total, PAGE, D), dg, device)
    q = _randn_f16((B, Hq, M, D), dg, device)
    w = PagedWorkload(
        name=name, q=q, k_pool=k_pool, v_pool=v_pool, block_table=bt.to(device),
        seqlen=torch.tensor(lengths, dtype=torch.int32, device=device),
        head_map=(torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(device),
        causal=causal, lengths=list(lengths))
    if q_offsets is not None:
        w.q_offsets = torch.tensor(q_offsets, dtype=torch.int32, device=device)
        w.q_offsets_host = list(q_offsets)
    if with_append:
        w.k_new = _randn_f16((B, Hk, 1, D), dg, device)
        w.v_new = _randn_f16((B, Hk, 1, D), dg, device)
        w.append_pos = torch.tensor([n - 1 for n in lengths], dtype=torch.int32, device=device)
    w.meta = dict(cfg=cfg_index, pool_pages=total, max_blocks=max_blocks, page_size=PAGE)
    return w


def _lengths(cfg_index, B, lo, hi):
    g = torch.Generator().manual_seed(1000 + cfg_index)
    return torch.randint(lo, hi + 1, (B,), generator=g).tolist()


def cfg1(device, dtype=torch.float16):
    """Contiguous causal MHA prefill: q, k, v [1, 8, 512, 64]."""
    g = _device_gen(device, 1001)
    shape = (1, 8, 512, 64)
    q, k, v = (torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)
               for _ in range(3))
    return q, k, v


def cfg2(device, B=4, S=2048):
    """Causal GQA prefill at the Qwen-32B shape over a paged, permuted pool."""
    return _paged("cfg2_prefill_qwen32b", 2, B, 40, 8, 128, S, [S] * B, True, device)


def cfg3(device, B=32):
    lengths = _lengths(3, B, 512, 8192)
    return _paged("cfg3_decode_qwen32b", 3, B, 40, 8, 128, 1, lengths, False, device,
                  max_blocks=8192 // PAGE)


def cfg4(device, B=64):
    """Decode + append: contexts U[1024, 16384]; the appended token is the last
    cached one, so seqlen = context + 1 and the pages hold room for it."""
    ctx = _lengths(4, B, 1024, 16384)
    lengths = [c + 1 for c in ctx]
    return _paged("cfg4_decode_append_llama70b", 4, B, 64, 8, 128, 1, lengths, False, device,
                  max_blocks=(16384 + 1 + PAGE - 1) // PAGE, with_append=True)


def cfg5(device, B=16, M=512):
    prior = _lengths(5, B, 0, 32768)
    lengths = [p + M for p in prior]
    return _paged("cfg5_chunked_prefill_llama70b", 5, B, 64, 8, 128, M, lengths, True, device,
                  max_blocks=(32768 + M + PAGE - 1) // PAGE, q_offsets=prior)


def cfg5_ragged(device, B=16, M=512):
    """cfg5 with ragged chunks (the per-sequence chunk schedule's steady state):
    the same priors as cfg5, but sequence b has only valid_b ~ U[64, M] live
    rows in its M-row chunk (q_lens), so seqlen_b = prior_b + valid_b. Timed
    with q_lens (padding rows skipped) and without (padding rows computed),
    both rated by the live rows' algorithmic flops."""
    prior = _lengths(5, B, 0, 32768)
    g = torch.Generator().manual_seed(1105)
    valid = torch.randint(64, M + 1, (B,), generator=g).tolist()
    lengths = [p + v for p, v in zip(prior, valid)]
    w = _paged("cfg5_ragged_chunked_prefill_llama70b", 5, B, 64, 8, 128, M, lengths, True, device,
               max_blocks=(32768 + M + PAGE - 1) // PAGE, q_offsets=prior)
    w.q_lens = torch.tensor(valid, dtype=torch.int32, device=device)
    w.q_lens_host = valid
    w.meta["live_rows"] = int(sum(valid))
    return w


# ------------------------------------------------------------------ costs ---

def visible_pairs(w: PagedWorkload) -> int:
    """Number of unmasked (query, key) pairs summed over heads."""
    tot = 0
    for b, n in enumerate(w.lengths):
        if not w.causal:
            tot += (w.q_lens_host[b] if w.q_lens_host is not None else w.M) * n
            continue
        qo = w.q_offsets_host[b] if w.q_offsets_host is not None else 0
        rows = w.q_lens_host[b] if w.q_lens_host is not None else w.M
        for_rows = 0
        # row i sees min(n, qo + i + 1) keys (rows past q_lens are padding)
        for i in range(rows):
            for_rows += max(0, min(n, qo + i + 1))
        tot += for_rows
    return tot * w.Hq


def attention_flops(w: PagedWorkload) -> float:
    """4*D flops per visible (query, key) pair (QK^T and PV multiply-adds)."""
    return 4.0 * w.D * visible_pairs(w)


def decode_bytes(w: PagedWorkload) -> float:
    """Live K/V bytes + q read + o write + block-table entries + seqlen."""
    kv = sum(w.lengths) * w.Hk * w.D * 2 * 2
    qo = 2 * w.B * w.Hq * w.M * w.D * 2
    bt = sum((n + PAGE - 1) // PAGE for n in w.lengths) * 4
    return float(kv + qo + bt + 4 * w.B)


def append_bytes(w: PagedWorkload) -> float:
    """K and V rows read once and written once."""
    return float(2 * 2 * w.B * w.Hk * w.D * 2)


def causal_flops_contiguous(B, H, M, N, D, q_offset=0):
    pairs = sum(max(0, min(N, q_offset + i + 1)) for i in range(M))
    return 4.0 * D * B * H * pairs


def roofline_peaks():
    """MI355X published peaks: HBM bytes/s and dense fp16 MFMA flop/s."""
    return dict(hbm=8.0e12, mfma_f16=2.5e15)


def sample_meta(w: PagedWorkload) -> dict:
    return dict(B=w.B, Hq=w.Hq, Hk=w.Hk, M=w.M, D=w.D,
                kv_tokens=int(sum(w.lengths)), min_len=int(min(w.lengths)),
                max_len=int(max(w.lengths)), **w.meta)


__all__ = ["PagedWorkload", "cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "cfg5_ragged", "attention_flops",
           "decode_bytes", "append_bytes", "causal_flops_contiguous", "roofline_peaks",
           "visible_pairs", "sample_meta"]
