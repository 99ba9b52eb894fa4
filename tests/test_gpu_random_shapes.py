"""Seeded random sweep of flash_attn_paged shapes against the fp64 oracle.

Each case draws batch size, head counts (GQA group 1..8), head dim, query
rows (decode and prefill paths), causal flag, per-sequence or scalar query
offsets, page size (multiples of 16 for the DMA kernels, others for the
register-staged kernel), sequence lengths (empty, partial pages, beyond the
written range) and a permuted block table over a shared pool whose dead slots
hold NaN. The bar is the usual elementwise tolerance against fp64.
"""
import random

import numpy as np
import pytest
import torch

from hrm_flashrenderer_amd import flash_attn_paged
from paged_ref import assert_close, paged_reference, poison_dead_slots, seeded

pytestmark = pytest.mark.gpu

CASES = 24


def _case(seed):
    r = random.Random(seed)
    D = r.choice([64, 128])
    Hk = r.choice([1, 2, 4])
    group = r.choice([1, 2, 4, 5, 8])
    Hq = Hk * group
    B = r.randint(1, 4)
    M = r.choice([1, 1, 2, 5, 16, 33, 64, 129, 200])
    PS = r.choice([16, 16, 32, 64, 128, 24, 8])
    causal = r.random() < 0.6 if M > 1 else r.random() < 0.2
    lengths = [r.choice([0, 1, 15, 16, 17, 100, 257, 600, 1000]) if r.random() < 0.2
               else r.randint(1, 1200) for _ in range(B)]
    if causal:
        # the chunk sits at the end of each sequence (chunked-prefill convention)
        offsets = [max(0, n - M) for n in lengths]
    else:
        offsets = [r.randint(0, 50) for _ in range(B)]
    return dict(D=D, Hk=Hk, Hq=Hq, B=B, M=M, PS=PS, causal=causal, lengths=lengths,
                offsets=offsets, per_seq=r.random() < 0.5)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_paged_shapes(gpu, seed):
    c = _case(seed)
    B, Hq, Hk, M, D, PS = c["B"], c["Hq"], c["Hk"], c["M"], c["D"], c["PS"]
    g = torch.Generator().manual_seed(seed)
    pages = [max(1, -(-n // PS)) for n in c["lengths"]]
    total = sum(pages) + 3
    perm = torch.randperm(total, generator=g).to(torch.int32)
    max_blocks = max(pages) + 1
    bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    kp = seeded((1, Hk, total, PS, D), 1000 + seed)
    vp = seeded((1, Hk, total, PS, D), 2000 + seed)
    poison_dead_slots(kp, vp, bt, c["lengths"], PS)
    q = seeded((B, Hq, M, D), 3000 + seed)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
    seqlen = torch.tensor(c["lengths"], dtype=torch.int32, device=gpu)
    if c["per_seq"] or len(set(c["offsets"])) > 1:
        qo = torch.tensor(c["offsets"], dtype=torch.int32, device=gpu)
        offsets = c["offsets"]
    else:
        qo = c["offsets"][0]
        offsets = [qo] * B
    out = flash_attn_paged(q, kp, vp, seqlen, PS, hm, c["causal"], qo,
                           block_table=bt.to(gpu)).cpu().numpy()
    ref = paged_reference(q, kp, vp, bt, c["lengths"], PS, hm, c["causal"], offsets)
    for (b, h), rr in ref.items():
        assert_close(out[b, h], rr, f"seed={seed} {c} b={b} h={h}")
