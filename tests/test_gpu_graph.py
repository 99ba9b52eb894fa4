"""Decode steps captured into a HIP graph (torch.cuda.graph): a serving loop
captures its per-token work once and replays it. Each replay, with new
inputs copied into the captured buffers and eager work and synchronizations
between replays, must give the eager call's output, pages and lengths bit for
bit. The captured calls state heads_per_kv, so nothing reads the head map
back to the host during capture."""
import pytest
import torch

from hrm_flashrenderer_amd import flash_attn_paged_append
from hrm_flashrenderer_amd.token_major import decode_token_major, workspace_bytes
from paged_ref import poison_dead_slots, seeded

pytestmark = pytest.mark.gpu


def _pool(gpu, B, Hk, D, lengths, extra, seed, PS=16):
    pages = [(n + extra + PS - 1) // PS for n in lengths]
    total = sum(pages) + 1
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    bt = torch.full((B, max(pages)), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    kp, vp = seeded((1, Hk, total, PS, D), seed + 1), seeded((1, Hk, total, PS, D), seed + 2)
    poison_dead_slots(kp, vp, bt, lengths, PS)
    return kp, vp, bt.to(gpu)


@pytest.mark.parametrize("rope", [False, True])
def test_decode_step_replayed_from_a_graph(gpu, rope):
    from hrm_flashrenderer_amd.rope import build_rope_cache
    B, Hq, Hk, D, steps = 6, 32, 8, 128, 3
    lengths = [1, 15, 16, 300, 1000, 2047]
    kp, vp, bt = _pool(gpu, B, Hk, D, lengths, steps, 700)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
    ropet = build_rope_cache(4096, D, device=gpu) if rope else None
    sl = torch.tensor(lengths, dtype=torch.int32, device=gpu)
    # the eager state and the graph's state start equal
    ke, ve, sle = kp.clone(), vp.clone(), sl.clone()
    q_s, k_s, v_s = seeded((B, Hq, 1, D), 710), seeded((B, Hk, 1, D), 711), seeded((B, Hk, 1, D), 712)

    def step(k_pages, v_pages, seqlen, q, k_new, v_new):
        return flash_attn_paged_append(q, k_pages, v_pages, k_new, v_new, seqlen, 16, hm,
                                       block_table=bt, rope=ropet, heads_per_kv=Hq // Hk)

    # warm up on a side stream (default priority) on throwaway copies, then capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(kp.clone(), vp.clone(), sl.clone(), q_s, k_s, v_s)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_s = step(kp, vp, sl, q_s, k_s, v_s)
    torch.cuda.synchronize()
    assert torch.equal(sl, sle), "capture must not run the step"

    for i in range(steps):
        q, k_new, v_new = (seeded((B, Hq, 1, D), 720 + i), seeded((B, Hk, 1, D), 730 + i),
                           seeded((B, Hk, 1, D), 740 + i))
        q_s.copy_(q)
        k_s.copy_(k_new)
        v_s.copy_(v_new)
        graph.replay()
        o_e = step(ke, ve, sle, q, k_new, v_new)
        torch.cuda.synchronize()
        assert torch.equal(o_s.view(torch.int16), o_e.view(torch.int16)), f"replay {i}: output"
        assert torch.equal(kp.view(torch.int16), ke.view(torch.int16)), f"replay {i}: K pages"
        assert torch.equal(vp.view(torch.int16), ve.view(torch.int16)), f"replay {i}: V pages"
        assert torch.equal(sl, sle), f"replay {i}: lengths"
        assert torch.equal(sl.cpu(), torch.tensor(lengths) + i + 1)
        assert not torch.isnan(o_s).any()


def test_token_major_step_replayed_from_a_graph(gpu):
    H, KVH, Dh, T = 40, 8, 128, 3000
    g = torch.Generator().manual_seed(760)
    k = torch.randn(T, KVH, Dh, generator=g).to(torch.float16).to(gpu)
    v = torch.randn(T, KVH, Dh, generator=g).to(torch.float16).to(gpu)
    ws = torch.empty(workspace_bytes(H, KVH, Dh, T - 1), dtype=torch.uint8, device=gpu)
    q_s = torch.randn(H, Dh, generator=g).to(gpu)
    t = 2500

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        decode_token_major(q_s, k, v, t, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_s = decode_token_major(q_s, k, v, t, workspace=ws)
    for i in range(3):
        q = torch.randn(H, Dh, generator=g).to(gpu)
        q_s.copy_(q)
        graph.replay()
        o_e = decode_token_major(q, k, v, t, workspace=torch.empty_like(ws))
        torch.cuda.synchronize()
        assert torch.equal(o_s, o_e), f"replay {i}"
