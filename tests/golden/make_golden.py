"""Write the golden vectors of the reference's CPU math path.

Run ONLY in the build container, where the reference is mounted read-only:
    python tests/golden/make_golden.py /root/reference

It loads the reference's flashattention_custom/ops.py by file path (the
module's `from . import _ext` then fails and it uses its pure-PyTorch math,
ops.py:7-12), runs it on small seeded inputs, and stores inputs and outputs in
tests/golden/ref_cpu_path.npz. Nothing else of the reference is read or kept;
the GPU box only sees the .npz. These vectors pin the bit-level behaviour of
oracle.attention.cpu_* (the CPU-baseline restatement): fp32 scores and
softmax, P rounded to the input dtype, P @ V in the input dtype.
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "ref_cpu_path.npz")


def load_reference_ops(ref_root: str):
    path = os.path.join(ref_root, "flashattention_custom", "ops.py")
    spec = importlib.util.spec_from_file_location("_reference_fa_ops", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert not mod._HAS_EXT, "reference extension must be absent (CPU math path)"
    return mod


def main(ref_root: str) -> None:
    ops = load_reference_ops(ref_root)
    rng = np.random.default_rng(20261201)
    out = {}

    def randn(*shape, dtype):
        return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dtype)

    # flash_attn (contiguous MHA), fp16 and fp32, causal with offsets and non-causal.
    cases = [
        ("attn_f16_causal", torch.float16, True, 0, 0, (1, 2, 16, 24, 64)),
        ("attn_f16_offset", torch.float16, True, 8, 0, (1, 2, 8, 24, 128)),
        ("attn_f32_causal", torch.float32, True, 0, 0, (1, 2, 16, 16, 64)),
        ("attn_f32_noncausal", torch.float32, False, 0, 0, (2, 1, 4, 20, 64)),
        ("attn_f16_kofs", torch.float16, True, 3, 5, (1, 1, 6, 12, 64)),
    ]
    for name, dt, causal, qo, ko, (B, H, M, N, D) in cases:
        q = randn(B, H, M, D, dtype=dt)
        k = randn(B, H, N, D, dtype=dt)
        v = randn(B, H, N, D, dtype=dt)
        o = ops.flash_attn(q, k, v, causal=causal, q_offset=qo, k_offset=ko)
        out[f"{name}/q"] = q.numpy()
        out[f"{name}/k"] = k.numpy()
        out[f"{name}/v"] = v.numpy()
        out[f"{name}/o"] = o.numpy()
        out[f"{name}/meta"] = np.array([int(causal), qo, ko], dtype=np.int64)

    # flash_attn_paged: GQA prefill chunk with q_offset, decode (M=1, non-causal).
    pcases = [
        # name, causal, q_offset, (B, Hq, Hk, M, P, PS, D), seqlen
        ("paged_prefill", True, 24, (2, 4, 2, 8, 3, 16, 128), [32, 29]),
        ("paged_decode", False, 0, (2, 4, 2, 1, 4, 16, 64), [17, 48]),
        ("paged_decode_mha", False, 0, (1, 3, 3, 1, 2, 8, 64), [11]),
    ]
    for name, causal, qo, (B, Hq, Hk, M, P, PS, D), seqlen in pcases:
        q = randn(B, Hq, M, D, dtype=torch.float16)
        kp = randn(B, Hk, P, PS, D, dtype=torch.float16)
        vp = randn(B, Hk, P, PS, D, dtype=torch.float16)
        sl = torch.tensor(seqlen, dtype=torch.int32)
        hm = (torch.arange(Hq) // (Hq // Hk)).to(torch.int32)
        o = ops.flash_attn_paged(q, kp, vp, sl, PS, hm, causal=causal, q_offset=qo, k_offset=0)
        for key, val in (("q", q), ("k_pages", kp), ("v_pages", vp), ("seqlen", sl),
                         ("head_map", hm), ("o", o)):
            out[f"{name}/{key}"] = val.numpy()
        out[f"{name}/meta"] = np.array([int(causal), qo, 0, PS], dtype=np.int64)

    # paged_kv_append: the reference test's page-crossing start, scaled down.
    B, Hk, P, PS, D, T, start = 2, 2, 3, 16, 64, 20, 13
    kp = randn(B, Hk, P, PS, D, dtype=torch.float16)
    vp = randn(B, Hk, P, PS, D, dtype=torch.float16)
    kn = randn(B, Hk, T, D, dtype=torch.float16)
    vn = randn(B, Hk, T, D, dtype=torch.float16)
    out["append/k_pages_in"] = kp.numpy().copy()
    out["append/v_pages_in"] = vp.numpy().copy()
    ops.paged_kv_append(kp, vp, kn, vn, start_pos=start, page_size=PS)
    out["append/k_new"] = kn.numpy()
    out["append/v_new"] = vn.numpy()
    out["append/k_pages_out"] = kp.numpy()
    out["append/v_pages_out"] = vp.numpy()
    out["append/meta"] = np.array([start, PS], dtype=np.int64)

    out["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
