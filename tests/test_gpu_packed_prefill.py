"""GPU parity of the packed-row prefill layout against the fp64 oracle.

With fewer than 128 query rows per q head (M < 128) and more rows per KV head
than one decode pass takes, the prefill kernel packs the (head, position) rows
of one KV head's q heads into shared 128-row tiles, so each KV head's pages
stream once for all of its q heads (for example 16 positions x 8 heads, the
M = 16 speculative-decode shape at 64/8 heads). The paged entry takes it when
the batch gives at least 256 such tiles (512 when one 64-row decode pass would
do); smaller batches stay on the decode kernels, whose multi-pass cases are in
test_gpu_attention.py. The contiguous entry always packs. The reference serves
every M with one kernel (csrc/flash_attn_sm75.cu:469-525); the bar is the
fp32-softmax tolerance |out - ref| <= 2e-3 + 1e-2*|ref|.

Covers one full tile, partly filled tiles, several tiles per KV head with
positions wrapping inside a wave, a head boundary inside a wave, D = 64,
q_lens padding rows, non-uniform and invalid head maps, a heads_per_kv bound
below the map's count, rotary queries, the contiguous GQA entry, and the
cfg4 pool at M = 16.
"""
import numpy as np
import pytest
import torch

from hrm_flashrenderer_amd import flash_attn, flash_attn_paged, workloads
from oracle import attention as ora
from paged_ref import assert_close, paged_reference, seeded
from test_gpu_attention import _run_and_check, _small_paged
from test_gpu_rope import _tables

pytestmark = pytest.mark.gpu

RAGGED = [700, 0, 150, 9, 333, 64, 1021, 40]


def _packed_batch(Hk, M, hpk):
    """Sequences enough for the paged entry to choose the packed layout."""
    rows = M * hpk
    tiles = (rows + 127) // 128
    need = 256 * (2 if rows <= 64 else 1)
    return -(-need // (Hk * tiles))


@pytest.mark.parametrize("Hq,Hk,M,D,causal", [
    (64, 8, 16, 128, True),     # 128 rows per KV head: one full tile
    (40, 8, 16, 128, True),     # 80 rows: one tile, 48 rows empty
    (64, 8, 24, 128, True),     # 192 rows: two tiles, positions wrap inside waves
    (16, 8, 100, 128, True),    # 200 rows of two heads: a head boundary inside a wave
    (64, 8, 8, 128, True),      # 64 rows: a half-filled tile (B = 64)
    (32, 4, 12, 64, False),     # D = 64, non-causal, 96 rows
    (48, 6, 16, 64, True),      # D = 64, 128 rows
])
def test_packed_rows(gpu, Hq, Hk, M, D, causal):
    """Every head of every sequence (ragged lengths, some empty or shorter
    than M) against the oracle, the query rows at the last M positions."""
    B = _packed_batch(Hk, M, Hq // Hk)
    lengths = [RAGGED[b % len(RAGGED)] + b for b in range(B)]
    lengths[1] = 0
    c = _small_paged(B, Hq, Hk, M, lengths, D=D, seed=900 + M + D + Hq, causal=causal,
                     q_offsets=[max(0, n - M) for n in lengths] if causal else None)
    _run_and_check(c, f"packed Hq={Hq} Hk={Hk} M={M} D={D} causal={causal} B={B}")


def test_packed_rows_match_per_head_tiles(gpu):
    """The packed layout against the one-q-head-per-tile layout of the same
    kernel (heads_per_kv <= 0 keeps it): equal within the tolerance, since the
    two differ only in which rows share a wave's lazy rescale."""
    B = 32
    lengths = [3000 - 91 * b for b in range(B)]
    c = _small_paged(B, 64, 8, 16, lengths, seed=950, causal=True,
                     q_offsets=[n - 16 for n in lengths])
    qo = torch.tensor(c["q_offsets"], dtype=torch.int32, device=gpu)
    args = (c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], True, 0, 0, qo, None,
            c["bt"], None, None, None)
    packed = torch.ops.hrm_fa.flash_attn_paged(*args, 8).cpu().numpy()
    per_head = torch.ops.hrm_fa.flash_attn_paged(*args, 0).cpu().numpy()
    assert_close(packed, per_head.astype(np.float64), "packed vs per-head tiles")


def test_packed_q_lens_padding_rows(gpu):
    """q_lens with packed rows: live rows match the oracle, padding rows are
    zeros even when their Q is NaN."""
    B, Hq, Hk, M = 32, 64, 8, 16
    q_lens = [[16, 0, 5, 9, 1][b % 5] for b in range(B)]
    prior = [[300, 40, 1000, 0, 77][b % 5] + b for b in range(B)]
    lengths = [p + n for p, n in zip(prior, q_lens)]
    lengths[1] = 50
    c = _small_paged(B, Hq, Hk, M, lengths, seed=960, causal=True, q_offsets=prior)
    for b, n in enumerate(q_lens):
        c["q"][b, :, n:] = float("nan")
    qo = torch.tensor(prior, dtype=torch.int32, device=gpu)
    ql = torch.tensor(q_lens, dtype=torch.int32, device=gpu)
    out = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], True, qo, 0,
                           block_table=c["bt"], q_lens=ql).cpu()
    qc = c["q"].clone()
    for b, n in enumerate(q_lens):
        qc[b, :, n:] = 0.0
        assert (out[b, :, n:] == 0).all(), f"padding rows of b={b}"
    ref = paged_reference(qc, c["kp"], c["vp"], c["bt"], lengths, 16, c["hm"], True, prior)
    for (b, h), r in ref.items():
        n = q_lens[b]
        assert_close(out[b, h, :n].numpy(), r[:n], f"packed q_lens b={b} h={h}")


@pytest.mark.parametrize("bound", [None, 3])
def test_packed_head_map_edges(gpu, bound):
    """A non-uniform head map (5, 3 and 2 heads per KV head) with two invalid
    entries: valid heads match the oracle in head-map order, invalid heads are
    NaN. With a heads_per_kv bound of 3 the heads past the third of KV head 2
    are NaN as well (nothing is written out of bounds)."""
    Hq, Hk, M = 12, 3, 40
    hm_list = [2, 0, 2, 1, 2, 0, 2, -1, 1, 7, 0, 2]
    B = _packed_batch(Hk, M, bound or 5)
    lengths = [60 + 7 * b for b in range(B)]
    c = _small_paged(B, Hq, Hk, M, lengths, seed=970, causal=True,
                     q_offsets=[n - M for n in lengths])
    c["hm"] = torch.tensor(hm_list, dtype=torch.int32, device=gpu)
    valid = [h for h, k in enumerate(hm_list) if 0 <= k < Hk]
    ref = paged_reference(c["q"], c["kp"], c["vp"], c["bt"], lengths, 16, c["hm"], True,
                          c["q_offsets"], pairs=[(b, h) for b in range(B) for h in valid])
    qo = torch.tensor(c["q_offsets"], dtype=torch.int32, device=gpu)
    if bound is None:
        out = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], True, qo,
                               0, block_table=c["bt"]).cpu().numpy()
        nan_heads = (7, 9)
    else:
        args = (c["q"], c["kp"], c["vp"], c["seqlen"], 16, c["hm"], True, 0, 0, qo, None,
                c["bt"], None, None, None)
        out = torch.ops.hrm_fa.flash_attn_paged(*args, bound).cpu().numpy()
        nan_heads = (7, 9, 6, 11)  # 6 and 11: the 4th and 5th heads of KV head 2
    for h in nan_heads:
        assert np.isnan(out[:, h]).all(), f"bound {bound} head {h}"
    for (b, h), r in ref.items():
        if h not in nan_heads:
            assert_close(out[b, h], r, f"head map bound {bound} b={b} h={h}")


@pytest.mark.parametrize("D", [64, 128])
def test_packed_rotary_queries(gpu, D):
    """Rotary queries (engine/rope.py:15-24) rotated in the packed kernel at
    their own positions, against fp64 attention over the oracle's rotated q."""
    B, Hq, Hk, M, PS = 32, 64, 8, 16, 16
    cos, sin = _tables(2048, D, gpu)
    lengths = [100 + 37 * b for b in range(B)]
    c = _small_paged(B, Hq, Hk, M, lengths, D=D, seed=990 + D, causal=True,
                     q_offsets=[n - M for n in lengths])
    qo = torch.tensor(c["q_offsets"], dtype=torch.int32, device=gpu)
    out = flash_attn_paged(c["q"], c["kp"], c["vp"], c["seqlen"], PS, c["hm"], True, qo, 0,
                           block_table=c["bt"], rope=(cos, sin)).cpu()
    qr = torch.empty_like(c["q"]).cpu()
    for b in range(B):
        pos = np.arange(c["q_offsets"][b], c["q_offsets"][b] + M)
        qr[b] = torch.from_numpy(ora.rope_f16(c["q"][b].cpu(), cos.cpu(), sin.cpu(), pos))
    ref = paged_reference(qr, c["kp"], c["vp"], c["bt"], lengths, PS, c["hm"], True,
                          c["q_offsets"], pairs=[(b, h) for b in (0, 13, 31) for h in range(Hq)])
    for (b, h), r in ref.items():
        assert_close(out[b, h].numpy(), r, f"packed rope D={D} b={b} h={h}")


@pytest.mark.parametrize("D", [64, 128])
def test_packed_contiguous_gqa(gpu, D):
    """flash_attn (contiguous K/V) with 8 q heads per KV head and M = 40: the
    rows of each KV head's q heads share tiles; per-sequence offsets."""
    B, Hq, Hk, M, N = 2, 16, 2, 40, 300
    q = seeded((B, Hq, M, D), 980 + D)
    k = seeded((B, Hk, N, D), 981 + D)
    v = seeded((B, Hk, N, D), 982 + D)
    qo = torch.tensor([N - M, 100], dtype=torch.int32, device=gpu)
    out = flash_attn(q, k, v, True, qo, 0).cpu()
    for b in range(B):
        ref = ora.attention_f64(q[b:b + 1].cpu(), k[b:b + 1].cpu(), v[b:b + 1].cpu(), True,
                                int(qo[b]), 0)
        assert_close(out[b:b + 1], ref, f"contiguous packed D={D} b={b}")


def test_packed_cfg4_pool_m16(gpu):
    """cfg4's pool (64 sequences of 1K-16K keys, 64/8 heads) with 16 query
    rows per sequence at its last positions, the query-row bench's M = 16
    case: sampled sequences, every head, against the fp64 oracle."""
    w = workloads.cfg4(gpu)
    M = 16
    g = torch.Generator(device=gpu)
    g.manual_seed(1204)
    q = torch.randn(w.B, w.Hq, M, w.D, generator=g, device=gpu).half()
    qo_host = [n - M for n in w.lengths]
    qo = torch.tensor(qo_host, dtype=torch.int32, device=gpu)
    out = flash_attn_paged(q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, True, qo,
                           block_table=w.block_table).cpu().numpy()
    assert np.isfinite(out).all()
    for b in (0, 21, 63):
        ref = paged_reference(q[b:b + 1], w.k_pool, w.v_pool, w.block_table[b:b + 1],
                              [w.lengths[b]], 16, w.head_map, True, [qo_host[b]])
        for (_, h), r in ref.items():
            assert_close(out[b, h], r, f"cfg4 M=16 b={b} h={h}")
