"""Host-side helpers of the GPU parity tests: fp64 references of paged
workloads (via the oracle), NaN poisoning of dead page slots, and tolerance
assertions. Imported by tests only."""
from __future__ import annotations

import math
from typing import Iterable, Optional, Sequence, Tuple

import numpy as np
import torch

from oracle import attention as ora

ATOL = 2e-3   # |out - ref| <= ATOL + RTOL * |ref| elementwise (fp32-softmax bar)
RTOL = 1e-2


def assert_close(out, ref, what=""):
    ok, worst = ora.within_tolerance(out, ref, ATOL, RTOL)
    assert ok, f"{what}: max(|out-ref| - {RTOL}|ref|) = {worst:.3e} > {ATOL}"


# The fp32 path (flash_attn with fp32 q/k/v) computes in fp32 throughout, so it
# is held to a bar two orders tighter: a regression that rounded P to fp16 or
# used a low-precision exponential (errors of 1e-4..1e-3) fails it.
ATOL_F32 = 1e-5
RTOL_F32 = 1e-4


def assert_close_f32(out, ref, what=""):
    ok, worst = ora.within_tolerance(out, ref, ATOL_F32, RTOL_F32)
    assert ok, f"{what}: max(|out-ref| - {RTOL_F32}|ref|) = {worst:.3e} > {ATOL_F32} (fp32 bar)"


def poison_dead_slots(k_pool, v_pool, block_table, lengths, page_size):
    """Write NaN into every pool slot that holds no live token, so a kernel
    that reads past seqlen (or an unmapped page) produces NaN outputs."""
    NB, Hk, P, PS, D = k_pool.shape
    live = torch.zeros(NB * P, PS, dtype=torch.bool)
    bt = block_table.cpu()
    for b, n in enumerate(lengths):
        npages = (n + page_size - 1) // page_size
        for p in range(npages):
            phi = int(bt[b, p])
            cnt = min(page_size, n - p * page_size)
            live[phi, :cnt] = True
    dead = (~live).view(NB, P, PS).to(k_pool.device)
    for pool in (k_pool, v_pool):
        pool.masked_fill_(dead.unsqueeze(1).unsqueeze(-1).expand(NB, Hk, P, PS, D), float("nan"))


def gather_seq(pool_cpu: torch.Tensor, bt_row: torch.Tensor, n: int, page_size: int):
    """[Hk, n, D] keys of one sequence from a host copy of the pool."""
    NB, Hk, P, PS, D = pool_cpu.shape
    npages = (n + page_size - 1) // page_size
    phys = bt_row[:npages].long()
    pages = pool_cpu[phys // P, :, phys % P]          # [npages, Hk, PS, D]
    return pages.transpose(0, 1).reshape(Hk, npages * PS, D)[:, :n]


def paged_reference(q, k_pool, v_pool, block_table, lengths, page_size, head_map, causal,
                    q_offsets=None, pairs: Optional[Iterable[Tuple[int, int]]] = None,
                    rows: Optional[slice] = None):
    """fp64 reference for (b, hq) pairs (default: all). Returns {(b, hq): [M', D]}."""
    qc = q.cpu()
    kc, vc = k_pool.cpu(), v_pool.cpu()
    bt = block_table.cpu()
    hm = head_map.cpu().tolist()
    B, Hq, M, D = qc.shape
    if pairs is None:
        pairs = [(b, h) for b in range(B) for h in range(Hq)]
    rows = rows or slice(0, M)
    i0 = rows.start or 0
    out = {}
    cache = {}
    for b, h in pairs:
        n = int(lengths[b])
        if b not in cache:
            cache = {b: (gather_seq(kc, bt[b], n, page_size), gather_seq(vc, bt[b], n, page_size))}
        ks, vs = cache[b]
        hk = hm[h]
        qo = int(q_offsets[b]) if q_offsets is not None else 0
        qq = qc[b, h, rows].numpy()[None, None]
        kk = ks[hk].numpy()[None, None]
        vv = vs[hk].numpy()[None, None]
        out[(b, h)] = ora.attention_f64(qq, kk, vv, causal, qo + i0, 0)[0, 0]
    return out


def decode_reference(w):
    """fp64 reference of a decode workload (all sequences and heads), grouping
    the q heads of one KV head into one matmul."""
    qc = w.q.cpu().double()
    kc, vc = w.k_pool.cpu(), w.v_pool.cpu()
    bt = w.block_table.cpu()
    B, Hq, M, D = qc.shape
    Hk = kc.shape[1]
    group = Hq // Hk
    out = np.zeros((B, Hq, M, D))
    scale = 1.0 / math.sqrt(D)
    for b in range(B):
        n = int(w.lengths[b])
        ks = gather_seq(kc, bt[b], n, 16).double()
        vs = gather_seq(vc, bt[b], n, 16).double()
        for hk in range(Hk):
            qg = qc[b, hk * group:(hk + 1) * group].reshape(group * M, D)
            s = (qg @ ks[hk].T) * scale
            s = s - s.max(dim=1, keepdim=True).values
            p = torch.exp(s)
            p = p / p.sum(dim=1, keepdim=True)
            out[b, hk * group:(hk + 1) * group] = (p @ vs[hk]).reshape(group, M, D).numpy()
    return out


def seeded(shape: Sequence[int], seed: int, dtype=torch.float16, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype).to(device)
