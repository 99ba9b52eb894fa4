"""fa_flash_attn_paged_fwd_noalloc, the entry point that allocates nothing,
through the C ABI: its outputs must equal fa_flash_attn_paged_fwd's (same
kernels; the decode partials live in the library's static scratch instead of
a caller workspace) on two calls in a row, the second smaller than the first
(the scratch keeps the first call's contents), on a prefill call (no
scratch), and on a second stream ordered after the first by an event. More
than 64 rows per KV head beyond the scratch run on the prefill kernel. (The
rejection of other shapes beyond the scratch needs no device and is tested in
test_boundary.py.)"""
import pytest
import torch

from hrm_flashrenderer_amd import _lib
from hrm_flashrenderer_amd.ops import heads_per_kv
from paged_ref import poison_dead_slots, seeded

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hk, M, lengths, seed, causal, PS=16):
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(seed)
    pages = [(n + PS - 1) // PS for n in lengths]
    total = sum(pages) + 3
    perm = torch.randperm(total, generator=g).to(torch.int32)
    bt = torch.full((B, max(pages) + 1), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    kp, vp = seeded((1, Hk, total, PS, 128), seed + 1), seeded((1, Hk, total, PS, 128), seed + 2)
    poison_dead_slots(kp, vp, bt, lengths, PS)
    q = seeded((B, Hq, M, 128), seed + 3)
    return dict(q=q, kp=kp, vp=vp, bt=bt.to(dev), PS=PS, causal=causal,
                seqlen=torch.tensor(lengths, dtype=torch.int32, device=dev),
                hm=(torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(dev),
                qo=torch.tensor([n - M for n in lengths], dtype=torch.int32, device=dev))


def _args(c, o):
    q, kp = c["q"], c["kp"]
    B, Hq, M, D = q.shape
    NB, Hk, P = kp.shape[:3]
    hpk = heads_per_kv(c["hm"], Hk)
    return ((q.data_ptr(), kp.data_ptr(), c["vp"].data_ptr(), c["seqlen"].data_ptr(), c["PS"],
             c["hm"].data_ptr(), o.data_ptr(), B, Hq, M, D, NB, Hk, P, int(c["causal"]), 0, 0,
             c["qo"].data_ptr() if c["causal"] else None, None, None, c["bt"].data_ptr(),
             c["bt"].size(1)), hpk, (B, Hq, M, D, Hk, c["bt"].size(1), c["PS"]))


def _both(c, stream=None):
    lib = _lib.load()
    stream = (stream or torch.cuda.current_stream()).cuda_stream
    o_ref, o_new = torch.empty_like(c["q"]), torch.empty_like(c["q"])
    a_ref, hpk, shape = _args(c, o_ref)
    ws_bytes = lib.fa_paged_workspace_bytes(*shape, hpk)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=c["q"].device)
    _lib.check(lib.fa_flash_attn_paged_fwd(*a_ref, hpk, ws.data_ptr(), ws_bytes, stream))
    a_new, _, _ = _args(c, o_new)
    _lib.check(lib.fa_flash_attn_paged_fwd_noalloc(*a_new, hpk, stream))
    torch.cuda.synchronize()
    return o_ref.cpu(), o_new.cpu(), ws_bytes


def _same(a, b):
    return torch.equal(torch.nan_to_num(a, nan=7.0), torch.nan_to_num(b, nan=7.0)) and \
        torch.equal(torch.isnan(a), torch.isnan(b))


def test_no_alloc_entry_matches_the_workspace_entry(gpu):
    g = torch.Generator().manual_seed(900)
    big = _case(64, 64, 8, 1, torch.randint(1024, 8192, (64,), generator=g).tolist(), 910, False)
    small = _case(5, 40, 8, 1, torch.randint(1, 900, (5,), generator=g).tolist(), 920, False)
    rows4 = _case(7, 16, 4, 4, torch.randint(4, 3000, (7,), generator=g).tolist(), 930, True)
    prefill = _case(3, 8, 2, 200, [600, 200, 333], 940, True)
    for name, c in (("decode B=64", big), ("decode B=5 after B=64", small), ("M=4", rows4),
                    ("prefill", prefill), ("decode B=5 again", small)):
        ref, new, ws_bytes = _both(c)
        assert (ws_bytes > 0) == (name != "prefill"), name
        assert _same(ref, new), name
        assert torch.isfinite(new).all(), name


def test_no_alloc_entry_on_a_second_stream(gpu):
    """Both entries launched on a second stream (default priority) that waits
    for the inputs made on the current stream, with the current stream
    waiting for the second one's results: the same outputs, bit for bit."""
    g = torch.Generator().manual_seed(960)
    c = _case(9, 32, 8, 1, torch.randint(100, 5000, (9,), generator=g).tolist(), 961, False)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ref, new, ws_bytes = _both(c, side)
    torch.cuda.current_stream().wait_stream(side)
    assert ws_bytes > 0
    assert _same(ref, new)
    assert torch.isfinite(new).all()


def test_no_alloc_entry_runs_many_rows_on_the_prefill_kernel(gpu):
    """256 query rows per KV head over two sequences: the workspace entry runs
    the decode kernels in four passes (its workspace is beyond the 32 MiB
    scratch); the allocation-free entry takes the prefill kernel instead, with
    the same results within the fp32-softmax tolerance."""
    from paged_ref import assert_close
    c = _case(2, 64, 8, 32, [3000, 777], 950, True)
    ref, new, ws_bytes = _both(c)
    assert ws_bytes > 32 << 20
    assert torch.isfinite(new).all()
    assert_close(new.numpy(), ref.double().numpy(), "no-alloc prefill vs decode passes")
