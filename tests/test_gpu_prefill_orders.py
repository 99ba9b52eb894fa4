"""GPU parity of the prefill grid's two work orders at full batch sizes.

A per-head prefill call without per-sequence q offsets runs its (sequence,
KV group) pairs in the natural per-XCD order; the same call with its q
offsets given as a per-sequence tensor ranks each XCD's pairs by key count
first (the chunked-prefill order). Each item's arithmetic is the same, so
the outputs must be bit-identical (NaN where the other has NaN), and both
are held to the fp64 oracle on sampled heads. Covered at 1024-2048 rows per
head and 24-40 q heads per sequence: causal and non-causal, D = 64 and 128,
q tiles cut short by M, sequences shorter than the chunk, an empty sequence,
an invalid head-map entry (NaN rows), padding rows (q_lens), rotary queries,
the contiguous operator, and launches back to back on two streams.
"""
import numpy as np
import pytest
import torch

from hrm_flashrenderer_amd import build_rope_cache, flash_attn, flash_attn_paged, workloads
from oracle import attention as ora
from paged_ref import assert_close, paged_reference, poison_dead_slots, seeded

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _same(a, b):
    return torch.equal(torch.nan_to_num(a, nan=7.0), torch.nan_to_num(b, nan=7.0)) and \
        torch.equal(torch.isnan(a), torch.isnan(b))


def _pool(B, Hk, D, lengths, seed, PS=16, cap_tokens=2048):
    g = torch.Generator().manual_seed(seed)
    pages = [(n + PS - 1) // PS for n in lengths]
    mb = cap_tokens // PS
    total = sum(pages) + 9
    perm = torch.randperm(total, generator=g).to(torch.int32)
    bt = torch.full((B, mb), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    kp, vp = seeded((1, Hk, total, PS, D), seed + 1), seeded((1, Hk, total, PS, D), seed + 2)
    poison_dead_slots(kp, vp, bt, lengths, PS)
    return kp, vp, bt.to(DEV)


@pytest.mark.parametrize("B,Hq,Hk,M,D,causal,lengths", [
    (4, 40, 8, 2048, 128, True, [2048] * 4),                 # cfg2's shape
    (2, 64, 8, 1536, 64, True, [1536, 1000]),                # D = 64, a short sequence
    (3, 32, 4, 2000, 128, False, [2000, 1777, 5]),           # partial last q tile
    (4, 48, 8, 1024, 128, True, [1024, 0, 700, 1024]),       # an empty sequence
])
def test_natural_and_ranked_orders_agree(gpu, B, Hq, Hk, M, D, causal, lengths):
    kp, vp, bt = _pool(B, Hk, D, lengths, 500 + M + D)
    q = seeded((B, Hq, M, D), 510 + M)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(DEV)
    sl = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    out = flash_attn_paged(q, kp, vp, sl, 16, hm, causal, block_table=bt)
    zeros = torch.zeros(B, dtype=torch.int32, device=DEV)
    plain = flash_attn_paged(q, kp, vp, sl, 16, hm, causal, zeros, block_table=bt)
    torch.cuda.synchronize()
    assert _same(out, plain), "natural and ranked orders differ"
    pairs = [(b, h) for b in range(B) for h in (0, Hq // 2 + 1, Hq - 1) if lengths[b] > 0]
    ref = paged_reference(q, kp, vp, bt, lengths, 16, hm, causal, None, pairs=pairs)
    on = out.cpu().numpy()
    for (b, h), r in ref.items():
        assert_close(on[b, h], r, f"b={b} h={h}")
    for b, n in enumerate(lengths):
        if n == 0:
            assert (on[b] == 0).all()


def test_orders_with_head_map_padding_and_rope(gpu):
    """A non-uniform head map with an entry outside [0, Hk) (NaN rows for
    that head), ragged live rows (q_lens: zero rows past them) and rotary
    queries, in both orders, bit for bit."""
    B, Hq, Hk, M, D = 3, 64, 8, 1024, 128
    lengths = [1024, 900, 333]
    kp, vp, bt = _pool(B, Hk, D, lengths, 620)
    q = seeded((B, Hq, M, D), 621)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32)
    hm[5] = 3
    hm[17] = 9     # outside [0, Hk): NaN rows
    hm = hm.to(DEV)
    sl = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    ql = torch.tensor([1024, 700, 333], dtype=torch.int32, device=DEV)
    rope = build_rope_cache(2048, D, device=DEV)
    zeros = torch.zeros(B, dtype=torch.int32, device=DEV)
    for kw in (dict(q_lens=ql), dict(rope=rope), dict(q_lens=ql, rope=rope)):
        out = flash_attn_paged(q, kp, vp, sl, 16, hm, True, block_table=bt, **kw)
        plain = flash_attn_paged(q, kp, vp, sl, 16, hm, True, zeros, block_table=bt, **kw)
        torch.cuda.synchronize()
        assert _same(out, plain), str(kw.keys())
        assert torch.isnan(out[:, 17, :300]).all()
        if "q_lens" in kw:
            assert (out[1, :, 700:] == 0).all() and (out[2, :, 333:] == 0).all()
        else:
            live = torch.ones(Hq, dtype=torch.bool)
            live[17] = False
            assert torch.isfinite(out[0, live]).all()
    out = flash_attn_paged(q, kp, vp, sl, 16, hm, True, block_table=bt).cpu().numpy()
    ref = paged_reference(q, kp, vp, bt, lengths, 16, hm, True, None,
                          pairs=[(0, 5), (1, 4), (2, 63)])
    for (b, h), r in ref.items():
        assert_close(out[b, h], r, f"b={b} h={h}")


@pytest.mark.parametrize("D", [64, 128])
def test_contiguous_operator_scalar_and_tensor_offsets(gpu, D):
    """flash_attn (contiguous K/V, GQA) at 1536 rows per head, against the
    same call with a per-sequence q offset tensor."""
    B, Hq, Hk, M = 2, 64, 8, 1536
    q, k, v = seeded((B, Hq, M, D), 700 + D), seeded((B, Hk, M, D), 701), seeded((B, Hk, M, D), 702)
    out = flash_attn(q, k, v, True)
    plain = flash_attn(q, k, v, True, torch.zeros(B, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert _same(out, plain)
    sel = [0, 37]
    ref = ora.attention_f64(q[:, sel].cpu(), k[:, [0, 4]].cpu(), v[:, [0, 4]].cpu(), True)
    assert_close(out[:, sel].cpu(), ref, f"contiguous D={D}")


def test_prefill_back_to_back_on_two_streams(gpu):
    """cfg2 three times in a row on the current stream and three times on a
    second stream: every output bit-identical to the first."""
    w = workloads.cfg2(DEV)
    first = flash_attn_paged(w.q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, True,
                             block_table=w.block_table)
    outs = [flash_attn_paged(w.q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, True,
                             block_table=w.block_table) for _ in range(3)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        outs += [flash_attn_paged(w.q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, True,
                                  block_table=w.block_table) for _ in range(3)]
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, first), f"launch {i + 1}"
    assert torch.isfinite(first).all()
