"""torch.library.opcheck of the custom ops the Python operators call: the
declared schemas (which arguments an op mutates, no aliasing of outputs and
inputs), the fake (meta) implementations that torch.compile and fake tensors
trace through, and AOT dispatch with dynamic shapes, each against a real run
on the device."""
import pytest
import torch

import hrm_flashrenderer_amd  # noqa: F401  (registers the hrm_fa ops)
from hrm_flashrenderer_amd.rope import build_rope_cache
from paged_ref import seeded

pytestmark = pytest.mark.gpu


def _paged_case(gpu, B=2, Hq=8, Hk=2, M=1, D=64, PS=16, lengths=(40, 17)):
    pages = [(n + PS) // PS for n in lengths]
    total = sum(pages) + 2
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    bt = torch.full((B, max(pages) + 1), -1, dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    kp = seeded((1, Hk, total, PS, D), 11)
    vp = seeded((1, Hk, total, PS, D), 12)
    q = seeded((B, Hq, M, D), 13)
    hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32).to(gpu)
    return dict(q=q, kp=kp, vp=vp, bt=bt.to(gpu), hm=hm, PS=PS,
                seqlen=torch.tensor(lengths, dtype=torch.int32, device=gpu),
                k_new=seeded((B, Hk, 1, D), 14), v_new=seeded((B, Hk, 1, D), 15))


def test_flash_attn_op(gpu):
    q, k, v = seeded((1, 8, 64, 64), 1), seeded((1, 2, 96, 64), 2), seeded((1, 2, 96, 64), 3)
    torch.library.opcheck(torch.ops.hrm_fa.flash_attn.default,
                          (q, k, v, True, 32, 0, None, None))
    qd = seeded((2, 8, 1, 64), 4)
    kd, vd = seeded((2, 2, 300, 64), 5), seeded((2, 2, 300, 64), 6)
    torch.library.opcheck(torch.ops.hrm_fa.flash_attn.default,
                          (qd, kd, vd, False, 299, 0, None, None))


def test_flash_attn_paged_op(gpu):
    c = _paged_case(gpu)
    cos, sin = build_rope_cache(128, 64, device=gpu)
    for rope in ((None, None), (cos, sin)):
        torch.library.opcheck(
            torch.ops.hrm_fa.flash_attn_paged.default,
            (c["q"], c["kp"], c["vp"], c["seqlen"], c["PS"], c["hm"], False, 0, 0, None, None,
             c["bt"], rope[0], rope[1]),
            {"q_lens": None, "heads_per_kv": 4})


def test_paged_kv_append_op(gpu):
    c = _paged_case(gpu)
    torch.library.opcheck(
        torch.ops.hrm_fa.paged_kv_append.default,
        (c["kp"], c["vp"], c["k_new"], c["v_new"], 0, c["seqlen"], c["PS"], c["bt"], None, None))


def test_flash_attn_paged_append_op(gpu):
    c = _paged_case(gpu)
    torch.library.opcheck(
        torch.ops.hrm_fa.flash_attn_paged_append.default,
        (c["q"], c["kp"], c["vp"], c["seqlen"], c["PS"], c["hm"], False, 0, None, c["bt"],
         c["k_new"], c["v_new"], True, 0, None, None, None),
        {"heads_per_kv": 4})


def test_paged_kv_scatter_op(gpu):
    c = _paged_case(gpu)
    positions = torch.tensor([[3], [9]], dtype=torch.int32, device=gpu)
    torch.library.opcheck(
        torch.ops.hrm_fa.paged_kv_scatter.default,
        (c["kp"], c["vp"], c["k_new"], c["v_new"], positions, c["PS"], c["bt"], None, None))
