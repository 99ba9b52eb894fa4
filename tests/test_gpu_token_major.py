"""Decode attention over the INT8 engine's token-major cache on the GPU
(attn_decode, scripts/deepseek_native_engine.sh:562-604, through the C entry
fa_decode_token_major): fp32 q, fp16 [T, KVH, Dh] caches, head map h % KVH by
default, against the fp64 oracle at the fp32-softmax tolerance. Rows past t
are NaN-poisoned, so a read beyond the attended keys shows up as NaN. Shapes
with an even KV-head count and at most 8 query heads per KV head run with
KV-head pairs per segment (40/8, 64/8, 32/32, 14/2 and the uneven head map);
12/3 and 72/8 run one KV head per segment."""
import math

import numpy as np
import pytest
import torch

from hrm_flashrenderer_amd.token_major import decode_token_major, workspace_bytes
from oracle import attention as ora
from paged_ref import assert_close

pytestmark = pytest.mark.gpu


def _case(T, KVH, Dh, H, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, Dh, generator=g, dtype=torch.float32)
    k = torch.randn(T, KVH, Dh, generator=g).to(torch.float16)
    v = torch.randn(T, KVH, Dh, generator=g).to(torch.float16)
    return q, k, v


# (12, 3): a KV-head count that does not divide the workgroup count evenly;
# (72, 8): 9 query heads per KV head.
@pytest.mark.parametrize("H,KVH,Dh", [(40, 8, 128), (64, 8, 128), (32, 32, 64), (14, 2, 64),
                                      (12, 3, 64), (72, 8, 128)])
@pytest.mark.parametrize("t", [0, 1, 15, 16, 17, 255, 1000, 4095])
def test_token_major_decode_matches_oracle(gpu, H, KVH, Dh, t):
    T = t + 9
    q, k, v = _case(T, KVH, Dh, H, 1000 + t + H, gpu)
    kd, vd = k.clone(), v.clone()
    kd[t + 1:] = float("nan")
    vd[t + 1:] = float("nan")
    out = decode_token_major(q.to(gpu), kd.to(gpu), vd.to(gpu), t).cpu()
    assert out.dtype == torch.float32 and out.shape == (H, Dh)
    ref = ora.decode_token_major_f64(q, k, v, t)
    assert_close(out, ref, f"H={H} KVH={KVH} Dh={Dh} t={t}")


def test_token_major_decode_head_map_scale_and_workspace_reuse(gpu):
    H, KVH, Dh, T = 40, 8, 128, 700
    q, k, v = _case(T, KVH, Dh, H, 77, gpu)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    ws = torch.empty(workspace_bytes(H, KVH, Dh, T - 1), dtype=torch.uint8, device=gpu)
    hm = [h // (H // KVH) for h in range(H)]  # the HF GQA mapping instead of h % KVH
    hm_d = torch.tensor(hm, dtype=torch.int32, device=gpu)
    for t, scale in ((T - 1, None), (300, 0.05), (5, 1.0 / math.sqrt(Dh))):
        out = decode_token_major(qd, kd, vd, t, scale=scale, head_map=hm_d, workspace=ws).cpu()
        ref = ora.decode_token_major_f64(q, k, v, t, scale=scale, head_map=hm)
        assert_close(out, ref, f"head_map t={t} scale={scale}")
    # out-of-range head map entries give NaN rows, the others stay exact
    bad = hm_d.clone()
    bad[3] = KVH
    out = decode_token_major(qd, kd, vd, 100, head_map=bad, workspace=ws).cpu()
    assert torch.isnan(out[3]).all()
    ref = ora.decode_token_major_f64(q, k, v, 100, head_map=[h if i != 3 else 0 for i, h in enumerate(hm)])
    keep = [i for i in range(H) if i != 3]
    assert_close(out[keep], ref[keep], "head map with one bad entry")


@pytest.mark.parametrize("t", [0, 33, 2500])
def test_token_major_decode_kv_head_pairs_uneven_map(gpu, t):
    """With an even KV-head count and at most 8 query heads per KV head, the
    decode segments serve KV heads in pairs (2j, 2j + 1), alternating their
    16-key groups. Here a head map gives KV head 0 seven query heads and its
    partner one (bound 7: 14 rows per pair), KV heads 2 and 3 one and six,
    and one entry is out of range (NaN row); the rest against the oracle."""
    H, KVH, Dh = 16, 4, 128
    hm = [0, 3, 0, 0, 1, 0, 3, 0, 3, 2, 0, 3, 9, 3, 0, 3]
    assert max(hm.count(k) for k in range(KVH)) == 7
    T = t + 20
    q, k, v = _case(T, KVH, Dh, H, 500 + t, gpu)
    kd, vd = k.clone(), v.clone()
    kd[t + 1:] = float("nan")
    vd[t + 1:] = float("nan")
    hm_d = torch.tensor(hm, dtype=torch.int32, device=gpu)
    out = decode_token_major(q.to(gpu), kd.to(gpu), vd.to(gpu), t, head_map=hm_d,
                             heads_per_kv=7).cpu()
    assert torch.isnan(out[12]).all()
    ref = ora.decode_token_major_f64(q, k, v, t, head_map=[h if h < KVH else 0 for h in hm])
    keep = [i for i in range(H) if i != 12]
    assert_close(out[keep], ref[keep], f"uneven head map t={t}")


def _large_logit_case(kind, T, KVH, Dh, H, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, Dh, generator=g, dtype=torch.float32)
    k = torch.randn(T, KVH, Dh, generator=g)
    v = torch.randn(T, KVH, Dh, generator=g).to(torch.float16)
    if kind == "x8":          # max |logit| about 40 (q ~ N(0, 64))
        q = q * 8
    elif kind == "x16":       # max |logit| about 75
        q = q * 16
    elif kind == "spikes":    # 4 dims with |q| in [100, 300], the rest N(0, 4)
        spikes = 100 + 200 * torch.rand(H, 4, generator=g)
        q = q * 2
        q[:, :4] = spikes * torch.sign(torch.randn(H, 4, generator=g))
    elif kind == "beyond_fp16":  # |q| up to ~1e5 (> 65504), keys ~1e-3: logits ~30
        q = q * 3e4
        k = k * 1e-3
    return q, k.to(torch.float16), v


# The engine computes q . k in fp32 (scripts/deepseek_native_engine.sh:573-577).
# At these logit sizes, rounding q to fp16 alone leaves errors of up to 2-5e-3
# beyond the 2e-3 + 1e-2|ref| bar (checked on the CPU against the same oracle).
# The kernel's hi/lo split of q passes. In the last case, q exceeds the fp16
# range, which the kernel's power-of-two prescale absorbs.
@pytest.mark.parametrize("kind", ["x8", "x16", "spikes", "beyond_fp16"])
@pytest.mark.parametrize("H,KVH,Dh", [(40, 8, 128), (64, 8, 128), (14, 2, 64)])
def test_token_major_decode_large_logits(gpu, kind, H, KVH, Dh):
    t = 4095
    T = t + 5
    q, k, v = _large_logit_case(kind, T, KVH, Dh, H, 5000 + H + Dh)
    kd, vd = k.clone(), v.clone()
    kd[t + 1:] = float("nan")
    vd[t + 1:] = float("nan")
    out = decode_token_major(q.to(gpu), kd.to(gpu), vd.to(gpu), t).cpu()
    assert torch.isfinite(out).all(), f"{kind}: non-finite output"
    ref = ora.decode_token_major_f64(q, k, v, t)
    assert_close(out, ref, f"{kind} H={H} KVH={KVH} Dh={Dh}")


def test_token_major_decode_rejects_bad_calls(gpu):
    q, k, v = _case(8, 2, 64, 4, 3, gpu)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    with pytest.raises(RuntimeError, match="outside the cache"):
        decode_token_major(qd, kd, vd, 8)
    with pytest.raises(RuntimeError, match="q must be fp32"):
        decode_token_major(qd.half(), kd, vd, 3)
    small = torch.empty(16, dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError, match="workspace of"):
        decode_token_major(qd, kd, vd, 3, workspace=small)


@pytest.mark.parametrize("seed", range(12))
def test_token_major_decode_random_shapes_and_maps(gpu, seed):
    """Seeded random shapes: KV-head counts 1-16 (even ones with at most 8
    query heads per KV head run on KV-head pairs, the others one KV head per
    segment), 1-12 query heads per KV head, D = 64 or 128, positions 0-6000,
    and every other case a random head map (some KV heads unused) passed
    with its exact bound; rows past t NaN-poisoned."""
    rng = np.random.default_rng(7100 + seed)
    KVH = int(rng.integers(1, 17))
    per = int(rng.integers(1, 13))
    H = KVH * per - int(rng.integers(0, per))  # not always a multiple of KVH
    Dh = int(rng.choice([64, 128]))
    t = int(rng.integers(0, 6001))
    T = t + 1 + int(rng.integers(0, 40))
    q, k, v = _case(T, KVH, Dh, H, 7200 + seed, gpu)
    kd, vd = k.clone(), v.clone()
    kd[t + 1:] = float("nan")
    vd[t + 1:] = float("nan")
    what = f"seed={seed} H={H} KVH={KVH} Dh={Dh} t={t}"
    if seed % 2:
        hm = [int(x) for x in rng.integers(0, KVH, size=H)]
        bound = max(hm.count(j) for j in range(KVH))
        hm_d = torch.tensor(hm, dtype=torch.int32, device=gpu)
        out = decode_token_major(q.to(gpu), kd.to(gpu), vd.to(gpu), t, head_map=hm_d,
                                 heads_per_kv=bound).cpu()
        ref = ora.decode_token_major_f64(q, k, v, t, head_map=hm)
        what += f" map bound={bound}"
    else:
        out = decode_token_major(q.to(gpu), kd.to(gpu), vd.to(gpu), t).cpu()
        ref = ora.decode_token_major_f64(q, k, v, t)
    assert torch.isfinite(out).all(), what
    assert_close(out, ref, what)
