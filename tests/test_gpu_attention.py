"""GPU parity of flash_attn / flash_attn_paged against the fp64 oracle.

Bar: |out - ref| <= 2e-3 + 1e-2*|ref| elementwise (the fp32-softmax tolerance),
NaN exactly where the reference yields NaN. Covers the reference's own
known-answer tests (flash_tests/test_kernel.py:28-66) at their shapes, all
five benchmark configurations (full size: every output for the decode
configs, sampled heads for the prefill configs), block tables over a
permuted shared pool with NaN-poisoned dead slots, per-sequence offsets,
GQA and arbitrary head maps, and the edge cases (no keys, fully masked rows,
invalid head-map entries, seqlen beyond capacity).
"""
import math
import os

import numpy as np
import pytest
import torch

from hrm_flashrenderer_amd import flash_attn, flash_attn_paged, paged_kv_append, workloads
from oracle import attention as ora
from paged_ref import (assert_close, assert_close_f32, decode_reference, paged_reference,
                       poison_dead_slots, seeded)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_cpu_path.npz")


def _identity_pages(k, PS):
    B, H, N, D = k.shape
    P = (N + PS - 1) // PS
    pages = torch.zeros(B, H, P, PS, D, dtype=k.dtype, device=k.device)
    pages.view(B, H, P * PS, D)[:, :, :N] = k
    return pages


# -------------------------------------------------- reference KAT shapes ----

@pytest.mark.parametrize("D", [64, 128])
def test_reference_kernel_kat(gpu, D):
    """flash_tests/test_kernel.py:33-64: B=1, H=8, M=128, N=256, PS=128; contiguous,
    paged (identity pages), and paged with q_offset=128, M=64."""
    torch.manual_seed(0)
    B, H, M, N, PS = 1, 8, 128, 256, 128
    q, k, v = seeded((B, H, M, D), 100 + D), seeded((B, H, N, D), 101 + D), seeded((B, H, N, D), 102 + D)
    out = flash_attn(q, k, v, causal=True, q_offset=0, k_offset=0)
    ref = ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), True)
    assert_close(out.cpu(), ref, "contiguous")
    kp, vp = _identity_pages(k, PS), _identity_pages(v, PS)
    seqlen = torch.tensor([N], dtype=torch.int32, device=gpu)
    hm = torch.arange(H, dtype=torch.int32, device=gpu)
    outp = flash_attn_paged(q, kp, vp, seqlen, PS, hm, causal=True, q_offset=0, k_offset=0)
    assert_close(outp.cpu(), ref, "paged")
    q2 = seeded((B, H, 64, D), 103 + D)
    outp2 = flash_attn_paged(q2, kp, vp, seqlen, PS, hm, causal=True, q_offset=128, k_offset=0)
    ref2 = ora.attention_f64(q2.cpu(), k.cpu(), v.cpu(), True, 128, 0)
    assert_close(outp2.cpu(), ref2, "paged offset")


def test_golden_reference_outputs(gpu):
    """GPU results are within tolerance of the reference CPU path's own outputs
    (tests/golden) and of the fp64 form on the same inputs."""
    g = np.load(GOLDEN, allow_pickle=False)
    for name in ("attn_f16_causal", "attn_f16_offset", "attn_f32_causal", "attn_f32_noncausal",
                 "attn_f16_kofs"):
        causal, qo, ko = g[f"{name}/meta"].tolist()
        q, k, v = (torch.from_numpy(g[f"{name}/{x}"]).to(gpu) for x in "qkv")
        out = flash_attn(q, k, v, bool(causal), qo, ko).cpu()
        check = assert_close_f32 if q.dtype == torch.float32 else assert_close
        check(out, ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), bool(causal), qo, ko), name)
        check(out, g[f"{name}/o"], name + " vs reference output")
    for name in ("paged_prefill", "paged_decode", "paged_decode_mha"):
        causal, qo, ko, ps = g[f"{name}/meta"].tolist()
        t = {x: torch.from_numpy(g[f"{name}/{x}"]).to(gpu)
             for x in ("q", "k_pages", "v_pages", "seqlen", "head_map")}
        out = flash_attn_paged(t["q"], t["k_pages"], t["v_pages"], t["seqlen"], ps, t["head_map"],
                               bool(causal), qo, ko).cpu()
        B = t["q"].size(0)
        kk = ora.gather_kv(g[f"{name}/k_pages"], B, ps)
        vv = ora.gather_kv(g[f"{name}/v_pages"], B, ps)
        ref = ora.attention_f64(g[f"{name}/q"], kk, vv, bool(causal), qo, ko,
                                kv_len=g[f"{name}/seqlen"], head_map=g[f"{name}/head_map"])
        assert_close(out, ref, name)
        assert_close(out, g[f"{name}/o"], name + " vs reference output")


# ------------------------------------------------------ contiguous path ----

@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_cfg1_causal_mha(gpu, dtype):
    q, k, v = workloads.cfg1(gpu, dtype)
    out = flash_attn(q, k, v)
    assert out.dtype == dtype and out.shape == q.shape
    check = assert_close_f32 if dtype == torch.float32 else assert_close
    check(out.cpu(), ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), True), f"cfg1 {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_contiguous_gqa_offsets_noncausal(gpu, dtype, D):
    B, Hq, Hk, M, N = 3, 6, 2, 77, 150
    q, k, v = seeded((B, Hq, M, D), 1, dtype), seeded((B, Hk, N, D), 2, dtype), seeded((B, Hk, N, D), 3, dtype)
    check = assert_close_f32 if dtype == torch.float32 else assert_close
    for causal, qo, ko in ((True, 0, 0), (True, 73, 0), (False, 0, 0), (True, 5, 9)):
        out = flash_attn(q, k, v, causal, qo, ko).cpu()
        check(out, ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), causal, qo, ko),
              f"{dtype} D={D} causal={causal} qo={qo} ko={ko}")
    qo_t = torch.tensor([0, 40, 73], dtype=torch.int32, device=gpu)
    out = flash_attn(q, k, v, True, qo_t, 0).cpu()
    check(out, ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), True, [0, 40, 73], 0),
          "per-sequence q_offset")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hk,M,N,causal,qo", [
    (40, 8, 1, 4097, False, 0),    # single-token decode, GQA 5 rows per K/V head
    (64, 8, 1, 1000, True, 999),   # causal decode at the last position
    (40, 8, 4, 777, True, 773),    # 4 positions x 5 heads = 20 rows per K/V head
    (8, 8, 4, 37, False, 0),       # MHA, short
    (8, 8, 2, 300, True, 150),     # rows that see part of the keys
])
def test_contiguous_decode_rows(gpu, D, Hq, Hk, M, N, causal, qo):
    """flash_attn with at most 32 query rows per K/V head runs on the split-K
    decode kernels (the call asks for a workspace); same bar against fp64."""
    from hrm_flashrenderer_amd import _lib
    B = 3
    lib = _lib.load()
    assert lib.fa_flash_attn_workspace_bytes(_lib.FA_DTYPE_F16, B, Hq, Hk, M, N, D) > 0
    q, k, v = seeded((B, Hq, M, D), 60 + M), seeded((B, Hk, N, D), 61), seeded((B, Hk, N, D), 62)
    out = flash_attn(q, k, v, causal, qo, 0).cpu()
    assert_close(out, ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), causal, qo, 0),
                 f"D={D} {Hq}/{Hk} M={M} N={N}")
    qo_t = torch.tensor([qo, max(qo - 5, 0), 3], dtype=torch.int32, device=gpu)
    out = flash_attn(q, k, v, True, qo_t, 0).cpu()
    assert_close(out, ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), True, qo_t.tolist(), 0),
                 "per-sequence q_offset")


def test_contiguous_decode_matches_prefill_kernel(gpu):
    """The same single-token calls through fa_flash_attn_fwd (prefill kernels,
    no workspace) and fa_flash_attn_fwd_ws (decode kernels): both within the
    bar of each other's fp64 reference and of each other."""
    from hrm_flashrenderer_amd import _lib
    lib = _lib.load()
    B, Hq, Hk, M, N, D = 4, 64, 8, 1, 2500, 128
    q, k, v = seeded((B, Hq, M, D), 70), seeded((B, Hk, N, D), 71), seeded((B, Hk, N, D), 72)
    o_pre, o_dec = torch.empty_like(q), torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.fa_flash_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o_pre.data_ptr(),
                                     0, B, Hq, Hk, M, N, D, 0, 0, 0, None, None, stream))
    nbytes = lib.fa_flash_attn_workspace_bytes(0, B, Hq, Hk, M, N, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    _lib.check(lib.fa_flash_attn_fwd_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                        o_dec.data_ptr(), 0, B, Hq, Hk, M, N, D, 0, 0, 0, None,
                                        None, ws.data_ptr(), nbytes, stream))
    torch.cuda.synchronize()
    ref = ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), False)
    assert_close(o_pre.cpu(), ref, "prefill kernels")
    assert_close(o_dec.cpu(), ref, "decode kernels")


def _many_sequences(B, Hq, Hk, D, lengths, seed, per_sequence=False, PS=16):
    g = torch.Generator().manual_seed(seed)
    pages = [(n + PS - 1) // PS for n in lengths]
    mb = max(pages) + 1
    if per_sequence:
        bt = torch.arange(B * mb, dtype=torch.int32).view(B, mb)
        NB, P = B, mb
    else:
        total = sum(pages) + 7
        perm = torch.randperm(total, generator=g).to(torch.int32)
        bt = torch.full((B, mb), -1, dtype=torch.int32)
        pos = 0
        for b, n in enumerate(pages):
            bt[b, :n] = perm[pos:pos + n]
            pos += n
        NB, P = 1, total
    kp, vp = seeded((NB, Hk, P, PS, D), seed + 1), seeded((NB, Hk, P, PS, D), seed + 2)
    poison_dead_slots(kp, vp, bt, lengths, PS)
    return kp, vp, bt


def _decode_rows_reference(q, kp, vp, bt, lengths, hm, PS=16):
    from paged_ref import gather_seq
    qc, kc, vc, hmc = q.cpu(), kp.cpu(), vp.cpu(), hm.cpu()
    out = np.zeros(tuple(q.shape))
    for b, n in enumerate(lengths):
        ks, vs = gather_seq(kc, bt[b], n, PS), gather_seq(vc, bt[b], n, PS)
        out[b] = ora.attention_f64(qc[b:b + 1], ks[None], vs[None], False, head_map=hmc)[0]
    return out


@pytest.mark.parametrize("per_sequence", [False, True])
def test_decode_batch_beyond_2048_sequences(gpu, per_sequence):
    """2100 sequences (more than one decode launch holds): the decode kernels
    run in launches of at most 2048 sequences; every row against fp64, over a
    shared permuted pool (block table) and over per-sequence pool rows (the
    reference's [B, Hk, P, PS, D] layout, no block table)."""
    B, Hq, Hk, D = 2100, 8, 2, 64
    g = torch.Generator().manual_seed(77)
    lengths = torch.randint(1, 81, (B,), generator=g).tolist()
    kp, vp, bt = _many_sequences(B, Hq, Hk, D, lengths, 7700, per_sequence)
    q = seeded((B, Hq, 1, D), 7710)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
    seqlen = torch.tensor(lengths, dtype=torch.int32, device=gpu)
    out = flash_attn_paged(q, kp, vp, seqlen, 16, hm, False,
                           block_table=None if per_sequence else bt.to(gpu))
    ref = _decode_rows_reference(q, kp, vp, bt, lengths, hm)
    assert_close(out.cpu().numpy(), ref, f"B={B} per_sequence={per_sequence}")


@pytest.mark.parametrize("rope", [False, True])
def test_fused_decode_step_beyond_2048_sequences(gpu, rope):
    """The fused decode step (advance mode) over 2100 sequences: output, pages
    and lengths bit for bit those of append + attention. Without rotary tables
    the decode kernels take the token; with them the rotary append runs first
    and each launch's combine kernel advances its slice of the lengths."""
    from hrm_flashrenderer_amd import flash_attn_paged_append
    from hrm_flashrenderer_amd.rope import build_rope_cache
    B, Hq, Hk, D = 2100, 8, 2, 64
    ropet = build_rope_cache(128, D, device=gpu) if rope else None
    g = torch.Generator().manual_seed(78)
    old = torch.randint(0, 64, (B,), generator=g).tolist()
    kp, vp, bt = _many_sequences(B, Hq, Hk, D, [n + 1 for n in old], 7800)
    poison_dead_slots(kp, vp, bt, old, 16)
    bt = bt.to(gpu)
    q = seeded((B, Hq, 1, D), 7810)
    k_new, v_new = seeded((B, Hk, 1, D), 7811), seeded((B, Hk, 1, D), 7812)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
    old_t = torch.tensor(old, dtype=torch.int32, device=gpu)
    kr, vr = kp.clone(), vp.clone()
    paged_kv_append(kr, vr, k_new, v_new, old_t, 16, block_table=bt, rope=ropet)
    o_ref = flash_attn_paged(q, kr, vr, old_t + 1, 16, hm, False, old_t, block_table=bt,
                             rope=ropet)
    sl = old_t.clone()
    o = flash_attn_paged_append(q, kp, vp, k_new, v_new, sl, 16, hm, False, old_t,
                                block_table=bt, rope=ropet)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(kp.view(torch.int16), kr.view(torch.int16))
    assert torch.equal(vp.view(torch.int16), vr.view(torch.int16))
    assert torch.equal(sl, old_t + 1)
    assert not torch.isnan(o).any()


def test_operators_under_inference_mode(gpu):
    """Head maps, pages and queries made under torch.inference_mode() (no
    version counters): the paged operators, the fused step and a stated
    heads_per_kv give the results of the same calls outside it."""
    from hrm_flashrenderer_amd import flash_attn_paged_append
    B, Hq, Hk, D = 3, 16, 4, 128
    lengths = [50, 300, 17]
    kp, vp, bt = _many_sequences(B, Hq, Hk, D, [n + 1 for n in lengths], 7900)
    q = seeded((B, Hq, 1, D), 7910)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
    seqlen = torch.tensor(lengths, dtype=torch.int32, device=gpu)
    bt = bt.to(gpu)
    ref = flash_attn_paged(q, kp, vp, seqlen, 16, hm, False, block_table=bt)
    with torch.inference_mode():
        hm_i = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
        assert hm_i.is_inference()
        out = flash_attn_paged(q, kp, vp, seqlen, 16, hm_i, False, block_table=bt)
        out_b = flash_attn_paged(q, kp, vp, seqlen, 16, hm_i, False, block_table=bt,
                                 heads_per_kv=Hq // Hk)
        k_i, v_i, sl_i = kp.clone(), vp.clone(), seqlen.clone()
        k_new, v_new = seeded((B, Hk, 1, D), 7920), seeded((B, Hk, 1, D), 7921)
        o_f = flash_attn_paged_append(q, k_i, v_i, k_new, v_new, sl_i, 16, hm_i, block_table=bt)
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(out_b, ref)
    kr, vr = kp.clone(), vp.clone()
    paged_kv_append(kr, vr, k_new, v_new, seqlen, 16, block_table=bt)
    o_r = flash_attn_paged(q, kr, vr, seqlen + 1, 16, hm, False, block_table=bt)
    assert torch.equal(o_f, o_r) and torch.equal(sl_i, seqlen + 1)
    assert torch.equal(k_i.view(torch.int16), kr.view(torch.int16))
    assert torch.equal(v_i.view(torch.int16), vr.view(torch.int16))


# ----------------------------------------------------------- paged path ----

def _small_paged(B, Hq, Hk, M, lengths, PS=16, D=128, seed=0, causal=True, q_offsets=None,
                 spare_pages=5, max_blocks=None):
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(seed)
    pages = [(n + PS - 1) // PS for n in lengths]
    total = sum(pages) + spare_pages
    perm = torch.randperm(total, generator=g).to(torch.int32)
    max_blocks = max(pages) + 2 if max_blocks is None else max_blocks
    bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    kp = seeded((1, Hk, total, PS, D), seed + 1)
    vp = seeded((1, Hk, total, PS, D), seed + 2)
    q = seeded((B, Hq, M, D), seed + 3)
    poison_dead_slots(kp, vp, bt, lengths, PS)
    return dict(q=q, kp=kp, vp=vp, bt=bt.to(dev), lengths=lengths,
                seqlen=torch.tensor(lengths, dtype=torch.int32, device=dev),
                hm=(torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(dev), PS=PS,
                causal=causal, q_offsets=q_offsets)


def _run_and_check(c, what, rows=None):
    qo = c["q_offsets"]
    qo_arg = 0 if qo is None else torch.tensor(qo, dtype=torch.int32, device=c["q"].device)
    out = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], c["PS"], c["hm"], c["causal"],
                           qo_arg, 0, block_table=c["bt"]).cpu().numpy()
    ref = paged_reference(c["q"], c["kp"], c["vp"], c["bt"], c["lengths"], c["PS"], c["hm"],
                          c["causal"], qo)
    for (b, h), r in ref.items():
        assert_close(out[b, h], r, f"{what} b={b} h={h}")
    return out


@pytest.mark.parametrize("D", [64, 128])
def test_paged_prefill_gqa_block_table(gpu, D):
    c = _small_paged(2, 10, 2, 300, [300, 300], D=D, seed=10 + D)
    _run_and_check(c, "prefill")


@pytest.mark.parametrize("capacity_blocks", [None, 300])
@pytest.mark.parametrize("D", [64, 128])
def test_prefill_tile_kernels_short_and_long_capacity(gpu, D, capacity_blocks):
    """The DMA prefill kernel with a block table of at most 4096 keys of
    capacity and with a wider one (300 pages of 16 = 4800 keys)."""
    prior = [0, 133, 0, 61]
    M = 200
    lengths = [p + M for p in prior]
    c = _small_paged(4, 8, 2, M, lengths, D=D, seed=40 + D, q_offsets=prior,
                     max_blocks=capacity_blocks)
    _run_and_check(c, f"causal cap={capacity_blocks}")
    c = _small_paged(3, 8, 2, 70, [200, 333, 97], D=D, seed=50 + D, causal=False,
                     max_blocks=capacity_blocks)
    _run_and_check(c, f"non-causal cap={capacity_blocks}")


def test_short_kernel_rows_past_one_page_table_fill(gpu):
    """Rows of 2048 < keys <= 4096 (the 32-key-tile kernel, whose per-wave page
    table covers 64 tiles per fill): the tiles past key 2048 come from a second
    fill of the table, with a permuted block table, causal with offsets and
    non-causal."""
    prior = [2900, 1990, 3500]
    M = 140
    lengths = [p + M for p in prior]
    c = _small_paged(3, 4, 1, M, lengths, seed=70, q_offsets=prior, max_blocks=256)
    _run_and_check(c, "causal rows past 2048 keys")
    c = _small_paged(2, 4, 2, 40, [4000, 2113], seed=71, causal=False, max_blocks=256)
    _run_and_check(c, "non-causal rows past 2048 keys")


def test_contiguous_long_rows(gpu):
    """Contiguous K/V longer than 4096 keys, causal with an
    offset and non-causal, N not a multiple of the tile."""
    B, Hq, Hk, M, N, D = 1, 4, 2, 96, 4203, 128
    q, k, v = seeded((B, Hq, M, D), 60), seeded((B, Hk, N, D), 61), seeded((B, Hk, N, D), 62)
    for causal, qo in ((True, N - M), (False, 0), (True, 2000)):
        out = flash_attn(q, k, v, causal, qo, 0).cpu()
        assert_close(out, ora.attention_f64(q.cpu(), k.cpu(), v.cpu(), causal, qo, 0),
                     f"long rows causal={causal} qo={qo}")


@pytest.mark.parametrize("B,Hq,Hk,M,seed", [(16, 8, 1, 64, 80), (6, 16, 4, 100, 81),
                                             (8, 64, 8, 128, 82), (72, 8, 8, 16, 83)])
def test_ragged_lengths_every_head(gpu, B, Hq, Hk, M, seed):
    """Sequences of different lengths whose (sequence, KV group) pairs divide
    over the 8 XCDs (2, 3 and 8 pairs per XCD, ordered by length with ties;
    72 per XCD, kept in index order): every head of every sequence is checked,
    so a pair run twice or never shows."""
    g = torch.Generator().manual_seed(seed)
    prior = torch.randint(0, 700, (B,), generator=g).tolist()
    prior[1] = prior[0]
    lengths = [p + M for p in prior]
    c = _small_paged(B, Hq, Hk, M, lengths, seed=seed, q_offsets=prior)
    _run_and_check(c, f"ragged B={B} Hq={Hq} Hk={Hk}")


@pytest.mark.parametrize("D,causal", [(128, False), (64, True), (64, False)])
def test_ragged_lengths_without_offsets(gpu, D, causal):
    """Prompts of different lengths in one prefill batch, no per-sequence
    offsets: the pairs spread over the XCDs in index order (2 pairs per XCD),
    every head of every sequence checked, with the rows past each sequence's
    length masked by causality or by its key count."""
    lengths = [200, 37, 256, 129, 1, 250, 64, 180]
    c = _small_paged(8, 16, 2, 256, lengths, D=D, seed=90 + D, causal=causal)
    _run_and_check(c, f"ragged D={D} causal={causal}")


@pytest.mark.parametrize("B,Hq,Hk", [(16, 8, 1), (8, 32, 8)])
def test_ragged_lengths_d64_sorted(gpu, B, Hq, Hk):
    """Chunked prefill at D=64 with per-sequence offsets (pairs ordered by
    length on each XCD)."""
    g = torch.Generator().manual_seed(95 + B)
    prior = torch.randint(0, 500, (B,), generator=g).tolist()
    lengths = [p + 96 for p in prior]
    c = _small_paged(B, Hq, Hk, 96, lengths, D=64, seed=96 + B, q_offsets=prior)
    _run_and_check(c, f"ragged D=64 B={B} Hq={Hq} Hk={Hk}")


@pytest.mark.parametrize("D", [64, 128])
def test_page_size_128_block_table(gpu, D):
    """The reference engine's default page size (engine/llama_tp.py:29) over a
    permuted pool: chunked prefill with per-sequence offsets (ordered by
    length per XCD) and ragged single-token decode, every head checked."""
    g = torch.Generator().manual_seed(97 + D)
    prior = torch.randint(0, 900, (8,), generator=g).tolist()
    M = 100
    c = _small_paged(8, 16, 2, M, [p + M for p in prior], PS=128, D=D, seed=98 + D,
                     q_offsets=prior)
    _run_and_check(c, f"PS=128 prefill D={D}")
    lengths = torch.randint(1, 1500, (8,), generator=g).tolist()
    c = _small_paged(8, 16, 2, 1, lengths, PS=128, D=D, seed=99 + D, causal=False)
    _run_and_check(c, f"PS=128 decode D={D}")


@pytest.mark.parametrize("M,PS,D,causal", [(300, 16, 128, True), (300, 16, 64, True),
                                             (200, 24, 128, True), (4, 16, 128, True),
                                             (4, 16, 128, False), (1, 16, 64, False)])
def test_q_lens_padding_rows(gpu, M, PS, D, causal):
    """q_lens: only rows i < q_lens[b] are live (a ragged chunk padded to M
    rows). Live rows match the oracle; padding rows are zeros even when their
    Q is NaN. Covers the tile-DMA prefill kernel (PS 16), the register-staged
    one (PS 24), and the decode kernels (M*group <= 64), with q_lens 0, M and
    partial tiles."""
    B, Hq, Hk = 5, 8, 2
    g = torch.Generator().manual_seed(300 + M + D + PS)
    q_lens = [M, 0, max(1, M // 3), max(1, M - 1), max(1, (M * 3) // 4)]
    prior = torch.randint(0, 400, (B,), generator=g).tolist()
    lengths = [p + n for p, n in zip(prior, q_lens)]
    lengths[1] = 50                      # keys but no live rows
    c = _small_paged(B, Hq, Hk, M, lengths, PS=PS, D=D, seed=310 + M + D, causal=causal,
                     q_offsets=prior if causal else None)
    for b, n in enumerate(q_lens):
        c["q"][b, :, n:] = float("nan")  # padding Q must never reach a live output
    qo = c["q_offsets"]
    qo_arg = 0 if qo is None else torch.tensor(qo, dtype=torch.int32, device=gpu)
    ql = torch.tensor(q_lens, dtype=torch.int32, device=gpu)
    out = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], PS, c["hm"], causal, qo_arg, 0,
                           block_table=c["bt"], q_lens=ql).cpu()
    qc = c["q"].clone()
    for b, n in enumerate(q_lens):
        qc[b, :, n:] = 0.0
        assert (out[b, :, n:] == 0).all(), f"padding rows of b={b}"
    ref = paged_reference(qc, c["kp"], c["vp"], c["bt"], lengths, PS, c["hm"], causal, qo)
    for (b, h), r in ref.items():
        n = q_lens[b]
        assert_close(out[b, h, :n].numpy(), r[:n], f"q_lens b={b} h={h}")


def test_chunked_prefill_per_sequence_offsets(gpu):
    prior = [0, 37, 150, 600]
    M = 130
    lengths = [p + M for p in prior]
    c = _small_paged(4, 8, 1, M, lengths, seed=20, q_offsets=prior)
    _run_and_check(c, "chunked prefill")


@pytest.mark.parametrize("Hq,Hk,lengths", [(40, 8, [512, 1000, 17, 2047]),
                                           (64, 8, [1025, 16, 3000]),
                                           (8, 8, [5, 700]), (32, 1, [300, 1])])
def test_decode_m1(gpu, Hq, Hk, lengths):
    c = _small_paged(len(lengths), Hq, Hk, 1, lengths, seed=30, causal=False)
    _run_and_check(c, f"decode {Hq}/{Hk}")


@pytest.mark.parametrize("B,Hq,Hk,seed", [(8, 64, 8, 31), (13, 40, 8, 32), (1, 64, 8, 33)])
def test_decode_combine_modes(gpu, B, Hq, Hk, seed):
    """Both combine layouts: up to 512 query rows merge with a workgroup per
    row (512 rows here; one 20000-key sequence, whose rows each gather many
    partial slots), more rows with a wave per row (520 rows)."""
    g = torch.Generator().manual_seed(seed)
    lengths = [20000] if B == 1 else torch.randint(1, 3000, (B,), generator=g).tolist()
    c = _small_paged(B, Hq, Hk, 1, lengths, seed=seed, causal=False)
    _run_and_check(c, f"decode rows={B * Hq}")


@pytest.mark.parametrize("lengths", [[0, 0, 9000, 0, 1, 0, 4000, 0, 15, 0],
                                     [0] * 30 + [20000] + [0] * 30 + [17, 0]])
def test_decode_cost_split_empty_segments(gpu, lengths):
    """The decode split charges every (sequence, KV head) segment, empty ones
    included, a fixed number of units once there are at least two units per
    workgroup (here 6000-10000 units over 512 workgroups): empty sequences
    around and between long ones must leave every row's slots where the
    combine kernel looks for them, and rows with no keys come out as zeros."""
    c = _small_paged(len(lengths), 40, 8, 1, lengths, seed=34, causal=False)
    out = _run_and_check(c, f"decode B={len(lengths)} with empty sequences")
    for b, n in enumerate(lengths):
        if n == 0:
            assert (out[b] == 0).all(), f"sequence {b} has no keys"


@pytest.mark.parametrize("length", [2032, 2048, 2049, 4112])
def test_decode_cost_split_thresholds(gpu, length):
    """One sequence, 8 KV heads: 8 * ceil(length / 16) units = 1016, 1024,
    1032 and 2056, on either side of the two-units-per-workgroup threshold
    (1024 with 512 workgroups) where the segment charge switches on, and
    where it is capped at units / (2 * workgroups)."""
    c = _small_paged(1, 64, 8, 1, [length], seed=35, causal=False)
    _run_and_check(c, f"decode length={length}")


@pytest.mark.parametrize("seed", [36, 37])
def test_decode_d64_ragged(gpu, seed):
    """Head size 64 through the decode kernels with segment charges on
    (about 6000 units over the device's workgroups)."""
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(0, 3000, (8,), generator=g).tolist()
    c = _small_paged(8, 64, 8, 1, lengths, D=64, seed=seed, causal=False)
    _run_and_check(c, f"decode D=64 lengths={lengths}")


@pytest.mark.parametrize("M,causal", [(2, True), (3, False), (4, True), (16, True)])
def test_decode_few_rows(gpu, M, causal):
    lengths = [400, 1500, 33]
    c = _small_paged(3, 40, 8, M, lengths, seed=40 + M, causal=causal,
                     q_offsets=[n - M for n in lengths] if causal else None)
    _run_and_check(c, f"M={M}")


@pytest.mark.parametrize("Hq,Hk,M,D,causal,ps", [
    (64, 8, 4, 128, True, 16),    # 32 rows per KV head: two row blocks in one K/V pass
    (64, 8, 8, 128, False, 16),   # 64 rows at D=128: four blocks in one pass
    (40, 8, 7, 128, True, 16),    # 35 rows: three live blocks of four
    (40, 8, 5, 128, True, 16),    # 25 rows: the second block half empty
    (64, 8, 8, 128, True, 24),    # per-row loads (page size 24): two passes of two blocks
    (32, 4, 8, 64, True, 16),     # 64 rows at D=64: four blocks in one pass
    (16, 4, 12, 64, False, 16),   # 48 rows: three live blocks of four
    (64, 8, 16, 128, True, 16),   # 128 rows, few sequences: two passes of four blocks
    (64, 8, 32, 128, True, 16),   # 256 rows: four passes
    (40, 8, 30, 64, True, 16),    # 150 rows at D=64: three passes, the last part-filled
])
def test_decode_row_blocks_per_pass(gpu, Hq, Hk, M, D, causal, ps):
    """The decode kernels serve up to 4 blocks of 16 query rows per pass over a
    KV head's pages (2 with per-row loads at D=128) and walk larger groups in
    passes (up to 256 rows per KV head when the batch is too small for the
    packed prefill layout); every head of every sequence is checked, with
    ragged lengths (one empty) and NaN-poisoned dead slots."""
    lengths = [700, 0, 1500, 33, 2100]
    c = _small_paged(5, Hq, Hk, M, lengths, PS=ps, D=D, seed=330 + M + D, causal=causal,
                     q_offsets=[max(0, n - M) for n in lengths] if causal else None)
    _run_and_check(c, f"row blocks Hq={Hq} Hk={Hk} M={M} D={D} PS={ps}")


@pytest.mark.parametrize("M", [1, 200])
def test_arbitrary_head_map(gpu, M):
    c = _small_paged(2, 6, 3, M, [700, 260], seed=50, causal=M > 1)
    c["hm"] = torch.tensor([2, 0, 2, 1, 2, 0], dtype=torch.int32, device=gpu)
    _run_and_check(c, "head_map")


def test_integration_shim_rejects_bad_dtypes_and_layouts(gpu):
    """The integration guide's `_ext` binding on device tensors: bf16, mixed
    dtypes and non-contiguous inputs raise the reference's messages before
    any C call (they would otherwise reach a kernel that reads them as fp16
    or fp32); a valid call through the real library matches flash_attn."""
    from test_boundary import _integration_shim_namespace
    ns = _integration_shim_namespace()
    q = seeded((1, 8, 64, 64), 700)
    with pytest.raises(RuntimeError, match="fp16 required"):
        ns["flash_attn_fwd"](q.bfloat16(), q.bfloat16(), q.bfloat16())
    with pytest.raises(RuntimeError, match="fp16 required"):
        ns["flash_attn_fwd"](q, q.float(), q)
    with pytest.raises(RuntimeError, match="contiguous required"):
        ns["flash_attn_fwd"](q.transpose(2, 3), q, q)
    kp = seeded((1, 2, 4, 16, 64), 701)
    sl = torch.tensor([50], dtype=torch.int32, device=gpu)
    hm = (torch.arange(8) // 4).to(torch.int32).to(gpu)
    with pytest.raises(RuntimeError, match="fp16 required"):
        ns["flash_attn_paged_fwd"](q.float(), kp, kp, sl, 16, hm)
    with pytest.raises(RuntimeError, match="seqlen int32 required"):
        ns["flash_attn_paged_fwd"](q, kp, kp, sl.long(), 16, hm)
    k1 = seeded((1, 2, 1, 64), 702)
    with pytest.raises(RuntimeError, match="fp16 required"):
        ns["paged_kv_append"](kp, kp, k1.bfloat16(), k1.bfloat16(), 0, 16)
    # with the real library: equal to the package's operators
    real = _integration_shim_namespace(real=True)
    k, v = seeded((1, 8, 64, 64), 703), seeded((1, 8, 64, 64), 704)
    assert torch.equal(real["flash_attn_fwd"](q, k, v), flash_attn(q, k, v))
    q1 = q[:, :, :1].contiguous()
    assert torch.equal(real["flash_attn_paged_fwd"](q1, kp, kp, sl, 16, hm, False),
                       flash_attn_paged(q1, kp, kp, sl, 16, hm, False))


def test_heads_per_kv_bound_on_the_decode_path(gpu):
    """The decode workspace holds heads_per_kv * M rows per KV head. A map that
    sends more heads to a KV head than the bound the caller states gets NaN
    rows for the heads past it (nothing is written out of bounds); the heads
    within it stay exact. The public operator derives the bound from the map."""
    c = _small_paged(2, 6, 3, 1, [700, 260], seed=51, causal=False)
    c["hm"] = torch.tensor([2, 0, 2, 1, 2, 0], dtype=torch.int32, device=gpu)  # 3 heads on KV 2
    ref = paged_reference(c["q"], c["kp"], c["vp"], c["bt"], c["lengths"], 16, c["hm"], False)
    args = (c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], False, 0, 0, None, None,
            c["bt"], None, None, None)
    for bound, nan_heads in ((2, [4]), (1, [2, 4, 5])):
        out = torch.ops.hrm_fa.flash_attn_paged(*args, bound).cpu().numpy()
        for (b, h), r in ref.items():
            if h in nan_heads:
                assert np.isnan(out[b, h]).all(), f"bound {bound} b={b} h={h}"
            else:
                assert_close(out[b, h], r, f"bound {bound} b={b} h={h}")
    out = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], False,
                           block_table=c["bt"]).cpu().numpy()
    for (b, h), r in ref.items():
        assert_close(out[b, h], r, f"derived bound b={b} h={h}")


@pytest.mark.parametrize("PS", [128, 24, 8])
def test_page_sizes_identity_layout(gpu, PS):
    """Reference layout [B, Hk, P, PS, D] without a block table."""
    B, Hq, Hk, D = 2, 4, 2, 128
    lengths = [3 * PS + 5, PS - 1]
    P = 4
    kp, vp = seeded((B, Hk, P, PS, D), 60), seeded((B, Hk, P, PS, D), 61)
    bt_id = torch.arange(B * P, dtype=torch.int32).view(B, P)   # identity map phi = b*P + p
    poison_dead_slots(kp, vp, bt_id, lengths, PS)
    seqlen = torch.tensor(lengths, dtype=torch.int32, device=gpu)
    hm = (torch.arange(Hq) // 2).to(torch.int32).to(gpu)
    for M, causal in ((1, False), (70, True)):
        q = seeded((B, Hq, M, D), 62 + M)
        qo = torch.tensor([n - M for n in lengths], dtype=torch.int32, device=gpu)
        out = flash_attn_paged(q, kp, vp, seqlen, PS, hm, causal, qo if causal else 0).cpu()
        for b in range(B):
            n = lengths[b]
            kk = kp[b].reshape(Hk, P * PS, D)[:, :n].cpu()[None]
            vv = vp[b].reshape(Hk, P * PS, D)[:, :n].cpu()[None]
            ref = ora.attention_f64(q[b:b + 1].cpu(), kk, vv, causal,
                                    int(qo[b]) if causal else 0, 0)
            assert_close(out[b:b + 1], ref, f"PS={PS} M={M} b={b}")


def test_edge_cases(gpu):
    B, Hq, Hk, PS, D = 3, 4, 2, 16, 128
    kp, vp = seeded((B, Hk, 4, PS, D), 70), seeded((B, Hk, 4, PS, D), 71)
    hm = torch.tensor([0, 1, 5, -1], dtype=torch.int32, device=gpu)   # heads 2, 3 invalid
    seqlen = torch.tensor([0, 40, 1000], dtype=torch.int32, device=gpu)  # 1000 > capacity 64
    for M, causal, ko in ((1, False, 0), (40, True, 0), (1, True, 50), (40, True, 50)):
        q = seeded((B, Hq, M, D), 72 + M)
        out = flash_attn_paged(q, kp, vp, seqlen, PS, hm, causal, 0, ko).cpu()
        assert torch.isnan(out[:, 2:]).all()
        assert (out[0, :2] == 0).all()                 # no keys -> zeros (ops.py semantics)
        for b in (1, 2):
            n = min(int(seqlen[b]), 64)
            kk = kp[b].reshape(Hk, 64, D)[:, :n].cpu()[None]
            vv = vp[b].reshape(Hk, 64, D)[:, :n].cpu()[None]
            ref = ora.attention_f64(q[b:b + 1, :2].cpu(), kk, vv, causal, 0, ko,
                                    head_map=[0, 1])
            assert_close(out[b:b + 1, :2], ref, f"edge M={M} causal={causal} ko={ko} b={b}")


def test_deterministic(gpu):
    c = _small_paged(2, 40, 8, 1, [5000, 3333], seed=80, causal=False)
    a = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], False,
                         block_table=c["bt"])
    b = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], False,
                         block_table=c["bt"])
    assert torch.equal(a, b)


# ------------------------------------------------ full-size configurations ----

@pytest.mark.parametrize("cfg", ["cfg3", "cfg4"])
def test_full_size_decode(gpu, cfg):
    w = getattr(workloads, cfg)(gpu)
    if w.k_new is not None:
        paged_kv_append(w.k_pool, w.v_pool, w.k_new, w.v_new, w.append_pos, 16,
                        block_table=w.block_table)
    poison_dead_slots(w.k_pool, w.v_pool, w.block_table, w.lengths, 16)
    out = flash_attn_paged(w.q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, False,
                           block_table=w.block_table).cpu().numpy()
    ref = decode_reference(w)
    assert_close(out, ref, cfg)


def _fp32_reference_all_pairs(w, out, what):
    """Every (sequence, head) output of a full-size prefill workload against an
    fp32 softmax reference computed on the GPU (torch fp32 matmuls, explicit
    causal mask): the BASELINE bar is stated against an fp32 softmax
    reference. The fp64 oracle checks sampled pairs on the CPU as well."""
    PS = 16
    B, Hq, M, D = w.q.shape
    Hk = w.Hk
    group = Hq // Hk
    scale = 1.0 / math.sqrt(D)
    bt = w.block_table
    worst = 0.0
    for b in range(B):
        n = w.lengths[b]
        npg = (n + PS - 1) // PS
        pages = bt[b, :npg].long()
        kk = w.k_pool[0][:, pages].reshape(Hk, npg * PS, D)[:, :n].float()
        vv = w.v_pool[0][:, pages].reshape(Hk, npg * PS, D)[:, :n].float()
        qo = w.q_offsets_host[b] if w.q_offsets_host is not None else 0
        rows = torch.arange(M, device=w.q.device)[:, None] + qo
        mask = torch.arange(n, device=w.q.device)[None, :] > rows          # [M, n]
        for hk in range(Hk):
            qq = w.q[b, hk * group:(hk + 1) * group].float()               # [group, M, D]
            sc = torch.matmul(qq, kk[hk].t().contiguous()) * scale          # [group, M, n]
            sc.masked_fill_(mask, float("-inf"))
            ref = torch.matmul(torch.softmax(sc, dim=-1), vv[hk])           # [group, M, D]
            got = out[b, hk * group:(hk + 1) * group].float()
            err = (got - ref).abs() - 1e-2 * ref.abs()
            worst = max(worst, float(err.max()))
            del sc, ref
    assert worst <= 2e-3, f"{what}: max(|out-ref| - 1e-2|ref|) = {worst:.3e} > 2e-3 (fp32 ref)"


def test_full_size_prefill_cfg2_sampled_heads(gpu):
    w = workloads.cfg2(gpu)
    out = flash_attn_paged(w.q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, True,
                           block_table=w.block_table).cpu().numpy()
    assert np.isfinite(out).all()
    # fp64 on the CPU: one q head of every (sequence, KV head) group, the head
    # within the group rotating, 32 of the 160 pairs
    group = w.Hq // w.Hk
    pairs = [(b, hk * group + (b + hk) % group) for b in range(w.B) for hk in range(w.Hk)]
    ref = paged_reference(w.q, w.k_pool, w.v_pool, w.block_table, w.lengths, 16, w.head_map,
                          True, None, pairs=pairs)
    for (b, h), r in ref.items():
        assert_close(out[b, h], r, f"cfg2 b={b} h={h}")
    _fp32_reference_all_pairs(w, torch.from_numpy(out).to(gpu), "cfg2 all 160 pairs")


def test_full_size_chunked_prefill_cfg5_sampled_heads(gpu):
    w = workloads.cfg5(gpu)
    poison_dead_slots(w.k_pool, w.v_pool, w.block_table, w.lengths, 16)
    out = flash_attn_paged(w.q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, True,
                           w.q_offsets, block_table=w.block_table).cpu().numpy()
    assert np.isfinite(out).all()
    # fp64 on the CPU: two q heads of every sequence, on KV heads b and b + 4
    # (mod 8) with the head within the group rotating, 32 of the 1024 pairs
    group = w.Hq // w.Hk
    pairs = [(b, hk * group + (3 * b + hk) % group) for b in range(w.B)
             for hk in sorted({b % w.Hk, (b + w.Hk // 2) % w.Hk})]
    ref = paged_reference(w.q, w.k_pool, w.v_pool, w.block_table, w.lengths, 16, w.head_map,
                          True, w.q_offsets_host, pairs=pairs)
    for (b, h), r in ref.items():
        assert_close(out[b, h], r, f"cfg5 b={b} h={h}")
    _fp32_reference_all_pairs(w, torch.from_numpy(out).to(gpu), "cfg5 all 1024 pairs")


# -------------------------------------------------- reference call pattern ----

def test_llama_tp_call_pattern_through_alias_package(gpu):
    """engine/llama_tp.py:59-78 and :171-200: append the chunk's K/V with one
    scalar start, set seqlen, then attend with causal=prefill and
    q_offset=start, through `flashattention_custom.ops` (the reference name)."""
    from flashattention_custom.ops import flash_attn_paged as fap, paged_kv_append as pka
    B, Hq, Hk, D, PS, P = 2, 8, 2, 128, 128, 4
    k_pages = torch.empty(B, Hk, P, PS, D, dtype=torch.float16, device=gpu)
    v_pages = torch.empty_like(k_pages)
    seqlen = torch.zeros(B, dtype=torch.int32, device=gpu)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
    ks, vs, outs, qs = [], [], [], []
    cur = 0
    for step, T in enumerate([200, 1, 1, 57]):
        q = seeded((B, Hq, T, D), 90 + step)
        k = seeded((B, Hk, T, D), 190 + step)
        v = seeded((B, Hk, T, D), 290 + step)
        pka(k_pages, v_pages, k, v, start_pos=cur, page_size=PS)
        cur += T
        seqlen.fill_(cur)
        out = fap(q=q, k_pages=k_pages, v_pages=v_pages, seqlen=seqlen, page_size=PS,
                  head_map=hm, causal=bool(T > 1), q_offset=cur - T, k_offset=0)
        ks.append(k), vs.append(v), outs.append(out), qs.append(q)
        kall = torch.cat(ks, dim=2).cpu()
        vall = torch.cat(vs, dim=2).cpu()
        ref = ora.attention_f64(q.cpu(), kall, vall, T > 1, cur - T, 0)
        assert_close(out.cpu(), ref, f"step {step}")
