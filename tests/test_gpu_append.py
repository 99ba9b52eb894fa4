"""GPU parity of paged_kv_append: bit-exact against the oracle's closed-form
index map (oracle.attention.append_f16), including the reference's own
known-answer case (flash_tests/test_append_fast.py:16-38)."""
import numpy as np
import pytest
import torch

from hrm_flashrenderer_amd import paged_kv_append, workloads
from oracle import attention as ora
from paged_ref import seeded

pytestmark = pytest.mark.gpu


def _bitexact(gpu_tensor, ref):
    return np.array_equal(gpu_tensor.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("init", ["zeros", "random"])
def test_append_reference_kat(gpu, init):
    B, Hk, P, PS, D, T, start = 2, 4, 8, 128, 128, 96, 128 + 17
    if init == "zeros":
        kp = torch.zeros(B, Hk, P, PS, D, dtype=torch.float16, device=gpu)
        vp = torch.zeros_like(kp)
    else:
        kp = seeded((B, Hk, P, PS, D), 1)
        vp = seeded((B, Hk, P, PS, D), 2)
    kn, vn = seeded((B, Hk, T, D), 3), seeded((B, Hk, T, D), 4)
    k_ref, v_ref = ora.append_f16(kp, vp, kn, vn, start, PS)
    paged_kv_append(kp, vp, kn, vn, start_pos=start, page_size=PS)
    torch.cuda.synchronize()
    assert _bitexact(kp, k_ref) and _bitexact(vp, v_ref)


@pytest.mark.parametrize("PS,D,T,start", [(16, 128, 1, 37), (24, 64, 40, 7), (128, 64, 300, 0),
                                          (1, 128, 5, 3), (16, 128, 33, 15)])
def test_append_page_sizes_and_head_dims(gpu, PS, D, T, start):
    B, Hk = 3, 2
    P = (start + T + PS - 1) // PS + 1
    kp, vp = seeded((B, Hk, P, PS, D), 5), seeded((B, Hk, P, PS, D), 6)
    kn, vn = seeded((B, Hk, T, D), 7), seeded((B, Hk, T, D), 8)
    k_ref, v_ref = ora.append_f16(kp, vp, kn, vn, start, PS)
    paged_kv_append(kp, vp, kn, vn, start, PS)
    torch.cuda.synchronize()
    assert _bitexact(kp, k_ref) and _bitexact(vp, v_ref)


def test_append_per_sequence_starts_with_block_table(gpu):
    B, Hk, PS, D, T = 6, 8, 16, 128, 3
    NP, max_blocks = 40, 6
    g = torch.Generator().manual_seed(11)
    bt = torch.randperm(NP, generator=g)[:B * max_blocks].view(B, max_blocks).to(torch.int32)
    bt[2, 4:] = -1                                   # unmapped tail pages of sequence 2
    starts = torch.tensor([0, 15, 62, 94, -2, 95], dtype=torch.int32)  # 95+3 > capacity 96
    kp, vp = seeded((1, Hk, NP, PS, D), 9), seeded((1, Hk, NP, PS, D), 10)
    kn, vn = seeded((B, Hk, T, D), 12), seeded((B, Hk, T, D), 13)
    k_ref, v_ref = ora.append_f16(kp, vp, kn, vn, starts.numpy(), PS, block_table=bt.numpy())
    paged_kv_append(kp, vp, kn, vn, starts.to(gpu), PS, block_table=bt.to(gpu))
    torch.cuda.synchronize()
    assert _bitexact(kp, k_ref) and _bitexact(vp, v_ref)


def test_append_full_size_decode_step(gpu):
    """cfg 4 (Llama-70B, B=64): one token per sequence at its own position; only
    those B*Hk rows change (checked via the written slots and a whole-pool
    checksum of everything else)."""
    w = workloads.cfg4(gpu)
    k_before = w.k_pool.clone()
    v_before = w.v_pool.clone()
    paged_kv_append(w.k_pool, w.v_pool, w.k_new, w.v_new, w.append_pos, 16,
                    block_table=w.block_table)
    torch.cuda.synchronize()
    bt = w.block_table.cpu()
    P = w.k_pool.size(2)
    changed = torch.zeros(P, 16, dtype=torch.bool)
    for b, n in enumerate(w.lengths):
        pos = n - 1
        phi = int(bt[b, pos // 16])
        changed[phi, pos % 16] = True
        assert torch.equal(w.k_pool[0, :, phi, pos % 16], w.k_new[b, :, 0])
        assert torch.equal(w.v_pool[0, :, phi, pos % 16], w.v_new[b, :, 0])
    keep = (~changed).to(gpu).view(1, 1, P, 16, 1)
    assert torch.equal(torch.where(keep, w.k_pool, 0), torch.where(keep, k_before, 0))
    assert torch.equal(torch.where(keep, w.v_pool, 0), torch.where(keep, v_before, 0))


def test_append_golden_reference_vectors(gpu):
    """The HIP kernel on the reference CPU path's own append vectors
    (tests/golden/ref_cpu_path.npz, written by flashattention_custom/ops.py:
    63-72 from these inputs): every page of both pools bit for bit."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_cpu_path.npz"),
                allow_pickle=False)
    start, ps = g["append/meta"].tolist()
    kp = torch.from_numpy(g["append/k_pages_in"]).to(gpu)
    vp = torch.from_numpy(g["append/v_pages_in"]).to(gpu)
    kn = torch.from_numpy(g["append/k_new"]).to(gpu)
    vn = torch.from_numpy(g["append/v_new"]).to(gpu)
    paged_kv_append(kp, vp, kn, vn, start, ps)
    torch.cuda.synchronize()
    assert _bitexact(kp, g["append/k_pages_out"]) and _bitexact(vp, g["append/v_pages_out"])
    # the same write with a per-sequence start tensor and an identity block table
    B, Hk, P = g["append/k_pages_in"].shape[:3]
    kp2 = torch.from_numpy(g["append/k_pages_in"]).to(gpu).reshape(1, B, Hk, P, ps, -1)
    kp2 = kp2.permute(0, 2, 1, 3, 4, 5).reshape(1, Hk, B * P, ps, -1).contiguous()
    vp2 = torch.from_numpy(g["append/v_pages_in"]).to(gpu).reshape(1, B, Hk, P, ps, -1)
    vp2 = vp2.permute(0, 2, 1, 3, 4, 5).reshape(1, Hk, B * P, ps, -1).contiguous()
    bt = torch.arange(B * P, dtype=torch.int32, device=gpu).view(B, P)
    starts = torch.full((B,), start, dtype=torch.int32, device=gpu)
    paged_kv_append(kp2, vp2, kn, vn, starts, ps, block_table=bt)
    torch.cuda.synchronize()
    back = lambda t: t.view(1, Hk, B, P, ps, -1).permute(0, 2, 1, 3, 4, 5).reshape(  # noqa: E731
        B, Hk, P, ps, -1)
    assert _bitexact(back(kp2), g["append/k_pages_out"])
    assert _bitexact(back(vp2), g["append/v_pages_out"])


def test_append_rejects_out_of_range_scalar_start(gpu):
    kp = torch.zeros(1, 1, 2, 16, 64, dtype=torch.float16, device=gpu)
    kn = torch.zeros(1, 1, 4, 64, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError, match="exceeds the page capacity"):
        paged_kv_append(kp, kp.clone(), kn, kn.clone(), 30, 16)
