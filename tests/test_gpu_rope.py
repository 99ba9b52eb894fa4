"""Fused rotary embedding (engine/rope.py:15-24) on the GPU.

* paged_kv_append(..., rope=(cos, sin)) writes exactly the oracle's
  rope_f16(k_new) (bit-exact) and copies V unchanged;
* flash_attn_paged(..., rope=(cos, sin)) equals attention over the oracle's
  rotated queries (tolerance bar), for prefill and decode, D = 64 and 128;
* positions outside the table: a scalar start or offset raises, per-sequence
  device starts write NaN keys.
"""
import numpy as np
import pytest
import torch

from hrm_flashrenderer_amd import flash_attn_paged, paged_kv_append
from hrm_flashrenderer_amd.kv_cache import PagedKVCache
from oracle import attention as ora
from paged_ref import assert_close, seeded

pytestmark = pytest.mark.gpu


def _tables(L, D, dev):
    cos, sin = ora.rope_tables(L, D)
    return torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)


@pytest.mark.parametrize("D", [64, 128])
def test_append_rope_bitexact(gpu, D):
    B, Hk, T, PS, P = 3, 2, 37, 16, 8
    cos, sin = _tables(300, D, gpu)
    kp = torch.zeros(B, Hk, P, PS, D, dtype=torch.float16, device=gpu)
    vp = torch.zeros_like(kp)
    k, v = seeded((B, Hk, T, D), 1), seeded((B, Hk, T, D), 2)
    paged_kv_append(kp, vp, k, v, 19, PS, rope=(cos, sin))          # scalar start
    kr = ora.rope_f16(k.cpu(), cos.cpu(), sin.cpu(), np.arange(19, 19 + T))
    want_k, want_v = ora.append_f16(np.zeros(kp.shape, np.float16), np.zeros(vp.shape, np.float16),
                                    kr, v.cpu().numpy(), 19, PS)
    assert np.array_equal(kp.cpu().numpy().view(np.uint16), want_k.view(np.uint16))
    assert np.array_equal(vp.cpu().numpy().view(np.uint16), want_v.view(np.uint16))
    # per-sequence starts through a block table over a shared pool
    starts = [0, 50, 91]
    pool_k = torch.zeros(1, Hk, 32, PS, D, dtype=torch.float16, device=gpu)
    pool_v = torch.zeros_like(pool_k)
    bt = torch.randperm(32, generator=torch.Generator().manual_seed(3))[:B * 10].view(B, 10)
    bt = bt.to(torch.int32).to(gpu)
    st = torch.tensor(starts, dtype=torch.int32, device=gpu)
    paged_kv_append(pool_k, pool_v, k, v, st, PS, block_table=bt, rope=(cos, sin))
    kr = np.stack([ora.rope_f16(k[b].cpu(), cos.cpu(), sin.cpu(), np.arange(s, s + T))
                   for b, s in enumerate(starts)])
    want_k, want_v = ora.append_f16(np.zeros(pool_k.shape, np.float16),
                                    np.zeros(pool_v.shape, np.float16), kr, v.cpu().numpy(),
                                    starts, PS, bt.cpu().numpy())
    assert np.array_equal(pool_k.cpu().numpy().view(np.uint16), want_k.view(np.uint16))
    assert np.array_equal(pool_v.cpu().numpy().view(np.uint16), want_v.view(np.uint16))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("M,causal", [(1, False), (3, True), (40, True), (150, True)])
def test_attention_with_rotary_queries(gpu, D, M, causal):
    """Cache appends with rotated keys, attention rotating q in the kernel,
    against fp64 attention over the oracle's rotated q and k (M = 40: the
    packed-row prefill layout, 160 rows per KV head)."""
    B, Hq, Hk, PS = 2, 8, 2, 16
    L = 2048
    cos, sin = _tables(L, D, gpu)
    cache = PagedKVCache(B, Hk, D, page_size=PS, device=gpu)
    prior = 300
    k0, v0 = seeded((B, Hk, prior, D), 10 + D), seeded((B, Hk, prior, D), 11 + D)
    cache.append(k0, v0, rope=(cos, sin))
    k1, v1 = seeded((B, Hk, M, D), 12 + D), seeded((B, Hk, M, D), 13 + D)
    cache.append(k1, v1, rope=(cos, sin))
    q = seeded((B, Hq, M, D), 14 + D)
    out = cache.attention(q, (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu), causal,
                          prior, rope=(cos, sin)).cpu()
    n = prior + M
    kall = torch.cat([k0, k1], dim=2).cpu()
    vall = torch.cat([v0, v1], dim=2).cpu()
    kr = ora.rope_f16(kall, cos.cpu(), sin.cpu(), np.arange(n))
    qr = ora.rope_f16(q.cpu(), cos.cpu(), sin.cpu(), np.arange(prior, prior + M))
    ref = ora.attention_f64(qr, kr, vall.numpy(), causal, prior, 0)
    assert_close(out, ref, f"rope D={D} M={M} causal={causal}")


def test_out_of_table_positions(gpu):
    D, B, Hk, PS = 128, 2, 1, 16
    cos, sin = _tables(64, D, gpu)
    kp = torch.zeros(B, Hk, 8, PS, D, dtype=torch.float16, device=gpu)
    vp = torch.zeros_like(kp)
    k = seeded((B, Hk, 4, D), 20)
    with pytest.raises(RuntimeError, match="outside the rotary table"):
        paged_kv_append(kp, vp, k, k, 62, PS, rope=(cos, sin))
    st = torch.tensor([0, 62], dtype=torch.int32, device=gpu)     # device starts: no check
    paged_kv_append(kp, vp, k, k, st, PS, rope=(cos, sin))
    rows = kp.cpu().view(B, Hk, 8 * PS, D)
    assert torch.isfinite(rows[0, :, :4].float()).all()
    assert torch.isfinite(rows[1, :, 62:64].float()).all()
    assert torch.isnan(rows[1, :, 64:66].float()).all()           # positions 64, 65 > table
    q = seeded((B, 4, 3, D), 21)
    sl = torch.tensor([4, 4], dtype=torch.int32, device=gpu)
    hm = torch.zeros(4, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="outside the rotary table"):
        flash_attn_paged(q, kp, vp, sl, PS, hm, True, 62, rope=(cos, sin))
