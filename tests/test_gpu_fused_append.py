"""GPU parity of the fused decode step (flash_attn_paged_append,
fa_flash_attn_paged_append_fwd) against the two calls it replaces.

The reference's decode step appends the new token (cache.append,
engine/llama_tp.py:65-78) and then runs flash_attn_paged over the cache
(:186-200). The fused call must give the same bits: the attention output,
every page of both pools (NaN-poisoned dead slots included, compared as raw
bits) and, in advance mode, the lengths. The new token's own slot holds NaN
before the step, so a kernel that read it from the pages instead of from
k_new / v_new would produce NaN rows. Both outputs are also held to the fp64
oracle at the fp32-softmax bar.

Shapes: 8 and 32 query rows per KV head (the fused decode kernels, in
advance mode: one and two 16-row blocks; with explicit positions the append
kernel runs first), 64 rows (decode kernels with four blocks, so the append
kernel runs first) and 128-row prefill chunks (prefill path); D = 64 and 128;
the rotary variant (the fused kernels rotate the new key); new tokens at
every place in a 16-key group and at page boundaries; an empty sequence (one
key after the step); in advance mode, a new token in an unmapped page,
causal rows that end before the new token, and pages of 24 tokens (the
decode kernels' per-row load variant).
"""
import pytest
import torch

from hrm_flashrenderer_amd import (PagedKVCache, build_rope_cache, flash_attn_paged,
                                   flash_attn_paged_append, paged_kv_append)
from paged_ref import assert_close, gather_seq, paged_reference, poison_dead_slots, seeded

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _setup(B, Hq, Hk, D, PS, old_lengths, seed, spare=6):
    """Pool over a permuted block table, mapped for old length + 1 tokens,
    slots past the old lengths NaN (the new token's slot included)."""
    g = torch.Generator().manual_seed(seed)
    new_lengths = [n + 1 for n in old_lengths]
    pages = [(n + PS - 1) // PS for n in new_lengths]
    total = sum(pages) + spare
    perm = torch.randperm(total, generator=g).to(torch.int32)
    mb = max(pages) + 1
    bt = torch.full((B, mb), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    kp = seeded((1, Hk, total, PS, D), seed + 1)
    vp = seeded((1, Hk, total, PS, D), seed + 2)
    poison_dead_slots(kp, vp, bt, old_lengths, PS)
    k_new = seeded((B, Hk, 1, D), seed + 3)
    v_new = seeded((B, Hk, 1, D), seed + 4)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(DEV)
    return kp, vp, bt.to(DEV), k_new, v_new, hm


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("advance", [False, True])
@pytest.mark.parametrize("Hq,Hk,M,D,causal,rope", [
    (64, 8, 1, 128, False, False),   # cfg4's step: 8 rows per KV head (fused, one block)
    (40, 8, 1, 128, False, True),    # cfg3's heads, rotary
    (32, 8, 8, 128, True, False),    # 32 rows per KV head (fused, two blocks)
    (16, 4, 1, 64, False, False),    # D = 64
    (16, 4, 8, 64, True, True),      # D = 64, two blocks, rotary
    (64, 8, 8, 128, True, False),    # 64 rows per KV head: append kernel, then decode
])
def test_fused_step_matches_append_then_attention(gpu, advance, Hq, Hk, M, D, causal, rope):
    PS = 16
    old = [0, 15, 16, 31, 100, 1000, 47]   # new token at group offsets 0, 15, 0, 15, 4, 8, 15
    B = len(old)
    seed = 9100 + Hq + 7 * M + D + int(rope) + 2 * int(advance)
    kp, vp, bt, k_new, v_new, hm = _setup(B, Hq, Hk, D, PS, old, seed)
    q = seeded((B, Hq, M, D), seed + 5)
    ropet = build_rope_cache(2048, D, device=DEV) if rope else None
    old_t = torch.tensor(old, dtype=torch.int32, device=DEV)
    new_t = old_t + 1
    # the query rows sit at the last M positions (row M-1 at the new token):
    # the causal limits and the rotary positions of q
    qo = torch.clamp(new_t - M, min=0)

    # reference: the two calls
    kr, vr = kp.clone(), vp.clone()
    paged_kv_append(kr, vr, k_new, v_new, old_t, PS, block_table=bt, rope=ropet)
    o_ref = flash_attn_paged(q, kr, vr, new_t, PS, hm, causal, qo, block_table=bt, rope=ropet)

    kf, vf = kp.clone(), vp.clone()
    if advance:
        sl = old_t.clone()
        o = flash_attn_paged_append(q, kf, vf, k_new, v_new, sl, PS, hm, causal, q_offset=qo,
                                    block_table=bt, rope=ropet)
    else:
        sl = new_t.clone()
        o = flash_attn_paged_append(q, kf, vf, k_new, v_new, sl, PS, hm, causal, qo,
                                    start_pos=old_t, block_table=bt, rope=ropet)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o), _bits(o_ref)), "output differs from append + attention"
    assert torch.equal(_bits(kf), _bits(kr)) and torch.equal(_bits(vf), _bits(vr)), "pages differ"
    assert torch.equal(sl, new_t)
    assert not torch.isnan(o).any()
    if not rope:
        ref = paged_reference(q, kr, vr, bt, [n + 1 for n in old], PS, hm, causal,
                              qo.tolist() if causal else None)
        on = o.cpu().numpy()
        for (b, h), r in ref.items():
            assert_close(on[b, h], r, f"b={b} h={h}")


@pytest.mark.parametrize("advance", [False, True])
def test_fused_step_prefill_path(gpu, advance):
    """128 query rows per sequence run on the prefill kernel: the append kernel
    runs first, then the attention sees the new token (and the advance)."""
    B, Hq, Hk, M, D, PS = 3, 8, 2, 128, 128, 16
    old = [200, 300, 511]
    kp, vp, bt, k_new, v_new, hm = _setup(B, Hq, Hk, D, PS, old, 9300 + int(advance))
    q = seeded((B, Hq, M, D), 9310)
    old_t = torch.tensor(old, dtype=torch.int32, device=DEV)
    new_t = old_t + 1
    qo = new_t - M
    kr, vr = kp.clone(), vp.clone()
    paged_kv_append(kr, vr, k_new, v_new, old_t, PS, block_table=bt)
    o_ref = flash_attn_paged(q, kr, vr, new_t, PS, hm, True, qo, block_table=bt)
    kf, vf = kp.clone(), vp.clone()
    sl = old_t.clone() if advance else new_t.clone()
    o = flash_attn_paged_append(q, kf, vf, k_new, v_new, sl, PS, hm, True, qo,
                                start_pos=None if advance else old_t, block_table=bt)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o), _bits(o_ref))
    assert torch.equal(_bits(kf), _bits(kr)) and torch.equal(_bits(vf), _bits(vr))
    assert torch.equal(sl, new_t)


def test_fused_step_scalar_position_and_unmapped_page(gpu):
    """A scalar position, and a per-sequence position whose page is not mapped
    (the append skips it, as paged_kv_append does, and the attention reads
    that position from the pool as the two calls would)."""
    B, Hq, Hk, D, PS = 4, 16, 2, 128, 16
    old = [63, 63, 63, 63]
    kp, vp, bt, k_new, v_new, hm = _setup(B, Hq, Hk, D, PS, old, 9400)
    q = seeded((B, Hq, 1, D), 9401)
    new_t = torch.full((B,), 64, dtype=torch.int32, device=DEV)
    kr, vr = kp.clone(), vp.clone()
    paged_kv_append(kr, vr, k_new, v_new, 63, PS, block_table=bt)
    o_ref = flash_attn_paged(q, kr, vr, new_t, PS, hm, False, block_table=bt)
    kf, vf = kp.clone(), vp.clone()
    o = flash_attn_paged_append(q, kf, vf, k_new, v_new, new_t.clone(), PS, hm, False, 0,
                                start_pos=63, block_table=bt)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o), _bits(o_ref)) and torch.equal(_bits(kf), _bits(kr))
    # sequence 2's new token in a page that is not mapped (entry -1): both
    # skip the write, and both read that page's keys as zeros
    bt2 = bt.clone()
    bt2[2, 3] = -1
    pos = torch.full((B,), 63, dtype=torch.int32, device=DEV)
    seq = new_t
    kr, vr = kp.clone(), vp.clone()
    paged_kv_append(kr, vr, k_new, v_new, pos, PS, block_table=bt2)
    o_ref = flash_attn_paged(q, kr, vr, seq, PS, hm, False, block_table=bt2)
    kf, vf = kp.clone(), vp.clone()
    o = flash_attn_paged_append(q, kf, vf, k_new, v_new, seq.clone(), PS, hm, False, 0,
                                start_pos=pos, block_table=bt2)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o), _bits(o_ref))
    assert torch.equal(_bits(kf), _bits(kr)) and torch.equal(_bits(vf), _bits(vr))


@pytest.mark.parametrize("rope", [False, True])
def test_cache_decode_steps_match_append_and_attention(gpu, rope):
    """PagedKVCache.decode_step, three steps in a row after a ragged prefill,
    against the cache's append() + attention() on a twin cache."""
    B, Hq, Hk, D = 5, 40, 8, 128
    ropet = build_rope_cache(4096, D, device=DEV) if rope else None
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(DEV)
    fused = PagedKVCache(B, Hk, D, page_size=16, device=DEV, max_seq_len=2048)
    twin = PagedKVCache(B, Hk, D, page_size=16, device=DEV, max_seq_len=2048)
    lengths = [1, 17, 100, 255, 640]
    k = seeded((B, Hk, max(lengths), D), 9500)
    v = seeded((B, Hk, max(lengths), D), 9600)
    for cache in (fused, twin):
        cache.append(k, v, None, rope=ropet, valid=lengths)   # ragged prompts from position 0
    for step in range(3):
        q = seeded((B, Hq, 1, D), 9700 + step)
        kn = seeded((B, Hk, 1, D), 9800 + step)
        vn = seeded((B, Hk, 1, D), 9900 + step)
        before = twin.seqlen.clone()
        twin.append(kn, vn, rope=ropet)
        o_ref = twin.attention(q, hm, False, before, rope=ropet)
        o = fused.decode_step(q, kn, vn, hm, rope=ropet)
        torch.cuda.synchronize()
        assert torch.equal(_bits(o), _bits(o_ref)), f"step {step}"
        assert fused.lengths == twin.lengths
        assert torch.equal(fused.seqlen, twin.seqlen)
    # every live row (slots no call wrote hold whatever the pool allocation held)
    for cache_pool, twin_pool in ((fused.k_pages, twin.k_pages), (fused.v_pages, twin.v_pages)):
        fc, tc = cache_pool.cpu(), twin_pool.cpu()
        fbt, tbt = fused.block_table.cpu(), twin.block_table.cpu()
        for b, n in enumerate(fused.lengths):
            a = gather_seq(fc, fbt[b], n, 16)
            r = gather_seq(tc, tbt[b], n, 16)
            assert torch.equal(_bits(a), _bits(r)), f"sequence {b}"


@pytest.mark.parametrize("rope", [False, True])
def test_fused_step_advance_edges(gpu, rope):
    """Advance mode (the fused kernels) at its edges, against append +
    attention: sequence 2's new token falls in an unmapped page (neither
    written nor substituted; both read that key from the pool), and with
    causal rows that end one position before the new token it is invisible
    (written, not attended)."""
    B, Hq, Hk, D, PS = 4, 16, 2, 128, 16
    old = [63, 40, 63, 7]
    kp, vp, bt, k_new, v_new, hm = _setup(B, Hq, Hk, D, PS, old, 9450)
    ropet = build_rope_cache(256, D, device=DEV) if rope else None
    bt[2, 3] = -1                      # position 63 of sequence 2: page 3
    old_t = torch.tensor(old, dtype=torch.int32, device=DEV)
    new_t = old_t + 1
    for causal, M, qo in ((False, 1, old_t), (True, 4, torch.clamp(old_t - 4, min=0))):
        q = seeded((B, Hq, M, D), 9451 + M)
        kr, vr = kp.clone(), vp.clone()
        paged_kv_append(kr, vr, k_new, v_new, old_t, PS, block_table=bt, rope=ropet)
        o_ref = flash_attn_paged(q, kr, vr, new_t, PS, hm, causal, qo, block_table=bt, rope=ropet)
        kf, vf, sl = kp.clone(), vp.clone(), old_t.clone()
        o = flash_attn_paged_append(q, kf, vf, k_new, v_new, sl, PS, hm, causal, q_offset=qo,
                                    block_table=bt, rope=ropet)
        torch.cuda.synchronize()
        what = f"causal={causal} M={M} rope={rope}"
        assert torch.equal(_bits(o), _bits(o_ref)), what
        assert torch.equal(_bits(kf), _bits(kr)) and torch.equal(_bits(vf), _bits(vr)), what
        assert torch.equal(sl, new_t), what


@pytest.mark.parametrize("D", [64, 128])
def test_fused_step_unaligned_pages(gpu, D):
    """Pages of 24 tokens (not a multiple of 16: the decode kernels' per-row
    load variant), advance mode, new tokens on both sides of page and group
    boundaries, against append + attention."""
    B, Hq, Hk, PS = 5, 16, 4, 24
    old = [0, 23, 24, 47, 200]
    kp, vp, bt, k_new, v_new, hm = _setup(B, Hq, Hk, D, PS, old, 9500 + D)
    q = seeded((B, Hq, 1, D), 9510 + D)
    old_t = torch.tensor(old, dtype=torch.int32, device=DEV)
    new_t = old_t + 1
    kr, vr = kp.clone(), vp.clone()
    paged_kv_append(kr, vr, k_new, v_new, old_t, PS, block_table=bt)
    o_ref = flash_attn_paged(q, kr, vr, new_t, PS, hm, False, block_table=bt)
    kf, vf, sl = kp.clone(), vp.clone(), old_t.clone()
    o = flash_attn_paged_append(q, kf, vf, k_new, v_new, sl, PS, hm, block_table=bt)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o), _bits(o_ref))
    assert torch.equal(_bits(kf), _bits(kr)) and torch.equal(_bits(vf), _bits(vr))
    assert torch.equal(sl, new_t)
    assert not torch.isnan(o).any()


@pytest.mark.parametrize("rope", [False, True])
def test_full_size_cfg4_fused_step(gpu, rope):
    """cfg4 at full size (B = 64, 64/8 heads, D = 128, contexts U[1024, 16384]
    over the permuted shared pool) as one fused step in advance mode, the call
    PagedKVCache.decode_step makes and the bench times. Output, both pools (as
    raw bits, NaN-poisoned dead slots and the new token's NaN slot included)
    and the lengths equal append + attention; every output row is held to
    the fp64 oracle. With rope, the oracle rotates q (at the new token's
    position) and the new key with the fp16 apply_rope restatement, and
    attends over the unrotated cached keys plus that rotated key."""
    import numpy as np

    from hrm_flashrenderer_amd import workloads
    from oracle import attention as ora
    from paged_ref import decode_reference

    w = workloads.cfg4(DEV)
    old = [n - 1 for n in w.lengths]            # contexts before the step
    bt = w.block_table
    poison_dead_slots(w.k_pool, w.v_pool, bt, old, 16)
    old_t = torch.tensor(old, dtype=torch.int32, device=DEV)
    ropet = None
    if rope:
        cos, sin = ora.rope_tables(16385, 128)
        ropet = (torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV))
    kr, vr = w.k_pool.clone(), w.v_pool.clone()
    paged_kv_append(kr, vr, w.k_new, w.v_new, old_t, 16, block_table=bt, rope=ropet)
    o_ref = flash_attn_paged(w.q, kr, vr, old_t + 1, 16, w.head_map, False, old_t,
                             block_table=bt, rope=ropet)
    sl = old_t.clone()
    o = flash_attn_paged_append(w.q, w.k_pool, w.v_pool, w.k_new, w.v_new, sl, 16, w.head_map,
                                block_table=bt, rope=ropet)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o), _bits(o_ref)), "output differs from append + attention"
    assert torch.equal(_bits(w.k_pool), _bits(kr)) and torch.equal(_bits(w.v_pool), _bits(vr))
    assert torch.equal(sl, old_t + 1)
    assert not torch.isnan(o).any()
    del kr, vr
    if rope:
        # the oracle's rotation of q and of the new key (the pool's other keys
        # are cached as they are), written into a host copy of the pool
        qc = ora.rope_f16(w.q.cpu(), cos, sin, np.array(old)[:, None, None])
        kn = ora.rope_f16(w.k_new.cpu(), cos, sin, np.array(old)[:, None, None])
        w.q = torch.from_numpy(qc)
        kpool = w.k_pool.cpu()
        btc = bt.cpu()
        for b, s in enumerate(old):
            phi = int(btc[b, s // 16])
            kpool[0, :, phi, s % 16] = torch.from_numpy(kn[b, :, 0])
        w.k_pool = kpool
    ref = decode_reference(w)
    assert_close(o.cpu().numpy(), ref, f"cfg4 fused step rope={rope}")
