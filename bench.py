#!/usr/bin/env python3
"""Benchmark of the MI355X attention path on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 2,4,3,5,5r,1,tm,gemm]
                    [--no-cpu-baseline]

Prints ONE JSON line on stdout (diagnostics go to stderr). The headline
`value` is causal GQA prefill TFLOP/s at configuration 2 (Qwen-32B shape,
B=4, S=2048, 40/8 heads, D=128, 16-token pages over a permuted pool): a step
is one flash_attn_paged call over the whole batch with K/V already paged in
HBM. The same line carries the decode half of the metric under "decode":
configuration 4 (Llama-70B shape, B=64, context U[1024,16384], 64/8 heads):
a step appends one token per sequence and then runs decode attention over the
full context; decode GB/s counts live K/V + q/o + block-table bytes.
Configurations 3, 5 and 1 are reported under "extra", with "5r" (cfg5 with
ragged chunks, timed with and without q_lens). "gemm" adds two vendor
references on the same GPU: an fp16 GEMM (hipBLASLt) and PyTorch's own flash
attention (SDPA, flash backend) on cfg2's shape.

Per-kernel durations come from HIP events recorded on the stream the kernels
run on (torch's current stream). `roofline.achieved` is algorithmic work per
launch / mean launch duration, the mean taken over the timed launches run back
to back between one event pair (`*_back_to_back`); a second pass with events
around every launch gives the spread (`kernel_ms`: p10, p90, ...). Before a
workload's warmup steps, 0.1 s of untimed launches let the shader clock
settle (see `settle`). The CPU baseline is the
oracle's restatement of the reference's CPU math path
(flashattention_custom/ops.py:34-72), timed on the host (kind "port").
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

from hrm_flashrenderer_amd import (build_rope_cache, flash_attn, flash_attn_paged,  # noqa: E402
                                   flash_attn_paged_append, paged_kv_append, workloads)
from hrm_flashrenderer_amd import _lib  # noqa: E402
from hrm_flashrenderer_amd.ops import heads_per_kv  # noqa: E402
from hrm_flashrenderer_amd.token_major import decode_token_major  # noqa: E402
from hrm_flashrenderer_amd.token_major import workspace_bytes as token_major_workspace  # noqa: E402

METRIC = "decode attn HBM GB/s + prefill TFLOP/s (fp16) on 1 MI355X; % of roofline"
PEAK_HBM_GBS = 8000.0
PEAK_MFMA_F16_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_info():
    model = platform.processor()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def timed(step, steps, warmup, marks=1):
    """Run `step(events)` warmup+steps times; `events` is a list of marks+1 events
    the step records between its launches. Returns (wall_s, [[ms per segment]...])."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(marks + 1)] for _ in range(steps)]
    t0 = time.perf_counter()
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    segs = [[e[i].elapsed_time(e[i + 1]) for i in range(marks)] for e in evs]
    del stream
    return wall, segs


SETTLE_S = 0.1


def settle(step, seconds=SETTLE_S):
    """Untimed launches for `seconds` of GPU time before a workload's warmup.
    From idle, the shader clock first boosts, then drops below its sustained
    level for some tens of launches, then settles (cfg2: about 193 us, then
    230-250 us, then 195-205 us per launch). The timed steps measure the
    settled state that a sustained load runs in."""
    step(None)  # the first call of a configuration may load code or allocate
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            step(None)
        torch.cuda.synchronize()


def back_to_back(step, steps, warmup):
    """Settle, run `step(None)` warmup+steps times with no events between the
    launches, and time the `steps` launches with one HIP event pair on the
    launching stream. Events recorded between launches leave a gap of a few
    microseconds on the GPU's timeline, which per-launch events would count;
    this is the mean duration the roofline uses. Returns (wall_s, mean_ms)."""
    stream = torch.cuda.current_stream()
    settle(step)
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step(None)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, e0.elapsed_time(e1) / steps


def dist(durs):
    """Summary of per-step kernel times in ms: mean, median, p10, p90, min, max."""
    v = sorted(durs)

    def q(f):
        return v[min(len(v) - 1, max(0, int(round(f * (len(v) - 1)))))]
    return {"mean": round(statistics.fmean(v), 4), "median": round(statistics.median(v), 4),
            "p10": round(q(0.1), 4), "p90": round(q(0.9), 4), "min": round(v[0], 4),
            "max": round(v[-1], 4)}


def roofline(bound, work, mean_ms, traffic=None):
    if bound == "hbm":
        achieved = work / (mean_ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    else:
        achieved = work / (mean_ms * 1e-3) / 1e12
        peak, unit = PEAK_MFMA_F16_TFLOPS, "TFLOP/s"
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# ---------------------------------------------------------------- configs ---

def bench_prefill(w, steps, warmup, traffic_key, traffic, q_lens=None):
    flops = workloads.attention_flops(w)
    qo = w.q_offsets if w.q_offsets is not None else 0
    stream = torch.cuda.current_stream()

    def step(ev):
        if ev:
            ev[0].record(stream)
        flash_attn_paged(w.q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, w.causal, qo,
                         block_table=w.block_table, q_lens=q_lens)
        if ev:
            ev[1].record(stream)

    wall, mean_ms = back_to_back(step, steps, warmup)
    _, segs = timed(step, steps, 0)
    durs = [s[0] for s in segs]
    return {
        "value": round(flops * steps / wall / 1e12, 2), "unit": "TFLOP/s",
        "ms_per_step": round(wall / steps * 1e3, 4),
        "kernel_ms_back_to_back": round(mean_ms, 4),
        "kernel_ms": dist(durs),
        "flops_per_step": flops,
        "roofline": roofline("mfma", flops, mean_ms, traffic.get(traffic_key)),
        "workload": workloads.sample_meta(w),
    }


def bench_decode(w, steps, warmup, traffic_key, traffic, rotate=None, rope=None):
    """Decode (+ append when the workload has new tokens). `rotate` is a second
    workload with its own pool, alternated per step to defeat the 256 MB MALL.
    `rope=(cos, sin)`: the fused rotary variant (keys rotated by the append, the
    query by the decode kernel)."""
    nbytes = workloads.decode_bytes(w)
    abytes = workloads.append_bytes(w) if w.k_new is not None else 0.0
    pools = [w] + ([rotate] if rotate is not None else [])
    stream = torch.cuda.current_stream()
    it = [0]

    def step(ev, append=True):
        x = pools[it[0] % len(pools)]
        it[0] += 1
        if ev:
            ev[0].record(stream)
        if append and x.k_new is not None:
            paged_kv_append(x.k_pool, x.v_pool, x.k_new, x.v_new, x.append_pos, 16,
                            block_table=x.block_table, rope=rope)
        if ev:
            ev[1].record(stream)
        flash_attn_paged(x.q, x.k_pool, x.v_pool, x.seqlen, 16, x.head_map, False,
                         x.append_pos if rope is not None else 0,
                         block_table=x.block_table, rope=rope)
        if ev:
            ev[2].record(stream)

    # whole steps back to back (the wall clock of `value`), then the decode
    # alone back to back (its mean is the roofline's; the append rewrites the
    # same token every step, so the cache is the same either way), then
    # per-step events for the distributions
    wall, mean_step = back_to_back(step, steps, warmup)
    _, mean_dec = back_to_back(lambda ev: step(ev, append=False), steps, 0)
    _, segs = timed(step, steps, 0, marks=2)
    dec = [s[1] for s in segs]
    app = [s[0] for s in segs]
    out = {
        "value": round(nbytes * steps / wall / 1e9, 2) if abytes == 0 else
        round((nbytes + abytes) * steps / wall / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(wall / steps * 1e3, 4),
        "decode_kernel_ms_back_to_back": round(mean_dec, 4),
        "decode_kernel_ms": dist(dec),
        "decode_bytes_per_step": nbytes,
        "roofline": roofline("hbm", nbytes, mean_dec, traffic.get(traffic_key)),
        "cache_defeat": "two pools alternated" if rotate is not None else
                        "pool larger than the 256 MB MALL",
        "workload": workloads.sample_meta(w),
    }
    if abytes:
        mean_app = statistics.fmean(app)
        out["append_kernel_ms"] = dist(app)
        out["append"] = roofline("hbm", abytes, mean_app, traffic.get("append"))
        out["append_bytes_per_step"] = abytes
        out["end_to_end_ms"] = round(mean_step, 4)
    return out


def bench_decode_fused(w, steps, warmup, two_call, rope=None):
    """cfg4's step (append one token per sequence, then decode) as one call,
    flash_attn_paged_append in advance mode: the decode kernel takes the new
    token from k_new / v_new and the merge kernel writes it into the pages,
    so the append has no launch of its own. `two_call` is bench_decode's
    result for the same workload (append kernel, then decode, at fixed
    lengths). GB/s counts the decode bytes, with the lengths' growth, and the
    append's bytes over the fused step."""
    stream = torch.cuda.current_stream()
    # The decode step as the cache takes it: each call appends at seqlen[b]
    # and advances it (the fused path), on a copy of the lengths before
    # cfg4's append. Each call adds one key per sequence, so the lengths are
    # reset before the warmup and before the per-launch pass, and
    # bytes_per_step counts the timed steps' mean growth (warmup + (steps -
    # 1) / 2 keys per sequence and KV head; a token past its sequence's mapped
    # pages is skipped, as the append kernel skips it).
    base = w.seqlen - 1
    lengths = base.clone()
    grow = warmup + (steps - 1) / 2
    grow_bytes = grow * w.B * w.Hk * w.D * 2 * 2
    nbytes = workloads.decode_bytes(w) + workloads.append_bytes(w) + grow_bytes

    def step(ev):
        if ev:
            ev[0].record(stream)
        flash_attn_paged_append(w.q, w.k_pool, w.v_pool, w.k_new, w.v_new, lengths, 16,
                                w.head_map, False, block_table=w.block_table, rope=rope)
        if ev:
            ev[1].record(stream)

    settle(step)
    lengths.copy_(base)
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step(None)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    mean_ms = e0.elapsed_time(e1) / steps
    lengths.copy_(base)
    _, segs = timed(step, steps, warmup)
    dec_ms = two_call["decode_kernel_ms_back_to_back"]
    return {
        "ms_per_step": round(wall / steps * 1e3, 4),
        "step_ms_back_to_back": round(mean_ms, 4),
        "step_ms": dist([x[0] for x in segs]),
        "bytes_per_step": nbytes,
        "roofline": roofline("hbm", nbytes, mean_ms),
        "two_call_step_ms_back_to_back": two_call["end_to_end_ms"],
        "decode_only_ms_back_to_back": dec_ms,
        "append_cost_us": round((mean_ms - dec_ms) * 1e3, 2),
        # the decode time scaled to the grown lengths' bytes taken off instead
        "append_cost_us_growth_corrected": round(
            (mean_ms - dec_ms * (1 + grow_bytes / workloads.decode_bytes(w))) * 1e3, 2),
        "append_cost_us_two_call": round((two_call["end_to_end_ms"] - dec_ms) * 1e3, 2),
    }


def bench_decode_rows(w, steps, warmup, rows=(1, 4, 8, 16)):
    """Paged attention over cfg4's pool with M query rows per sequence (the
    last M positions, causal: speculative or short-chunk decode). M = 1 and 4
    take the decode kernels; M = 8 and 16 (64 and 128 rows per KV head over
    64 sequences) take the prefill kernel's packed layout, which fills 128-row
    tiles with the (head, position) rows of one KV head (the library picks the
    path; `path` reports it). GB/s counts the live K/V, q/o, block table and
    seqlen bytes once."""
    res = {}
    dev = w.q.device
    g = torch.Generator(device=dev)
    g.manual_seed(1204)
    for M in rows:
        q = torch.randn(w.B, w.Hq, M, w.D, generator=g, device=dev).half()
        qo = torch.tensor([n - M for n in w.lengths], dtype=torch.int32, device=dev)
        nbytes = (sum(w.lengths) * w.Hk * w.D * 4 + 2 * w.B * w.Hq * M * w.D * 2
                  + sum((n + 15) // 16 for n in w.lengths) * 4 + 4 * w.B)

        def step(ev, q=q, qo=qo):
            flash_attn_paged(q, w.k_pool, w.v_pool, w.seqlen, 16, w.head_map, True, qo,
                             block_table=w.block_table)

        _, mean_ms = back_to_back(step, steps, warmup)
        ws = _lib.load().fa_paged_workspace_bytes(w.B, w.Hq, M, w.D, w.Hk, w.block_table.size(1),
                                                  16, heads_per_kv(w.head_map, w.Hk))
        res[f"M{M}"] = {"kernel_ms_back_to_back": round(mean_ms, 4), "bytes_per_step": nbytes,
                        "roofline": roofline("hbm", nbytes, mean_ms),
                        "path": "decode" if ws > 0 else "prefill (packed rows)"}
    return res


def bench_gemm_reference(dev, n=8192, iters=20):
    """fp16 GEMM of the vendor library (torch.matmul -> hipBLASLt) on the same
    GPU: the MFMA rate a plain GEMM sustains here, next to the published peak
    that roofline.peak uses. Reported only; not part of the attention path."""
    a = torch.randn(n, n, device=dev, dtype=torch.float16)
    b = torch.randn(n, n, device=dev, dtype=torch.float16)
    for _ in range(3):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        torch.matmul(a, b)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    tf = 2.0 * n ** 3 / ms / 1e9
    return {"tflops": round(tf, 1), "frac_of_peak": round(tf / PEAK_MFMA_F16_TFLOPS, 4), "ms": round(ms, 4),
            "shape": f"{n}x{n}x{n} fp16, fp32 accumulate", "library": "torch.matmul (hipBLASLt)"}


def bench_vendor_attention_reference(dev, iters=30):
    """PyTorch's own flash attention (scaled_dot_product_attention restricted
    to its flash backend, AOTriton on ROCm) on cfg2's shape as contiguous
    fp16 tensors (B=4, 40/8 heads, S=2048, D=128, causal, GQA), beside this
    library's contiguous entry on the same tensors; flops counted as for
    cfg2 (4*D per visible pair). Then the same for one decode row per
    sequence (the contiguous-decode extra's shape), in GB/s. Reported only;
    not part of the attention path. The math backend is never allowed: the
    call raises instead."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    import torch.nn.functional as F
    B, Hq, Hk, S, D = 4, 40, 8, 2048, 128
    flops = workloads.causal_flops_contiguous(B, Hq, S, S, D)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    q = torch.randn(B, Hq, S, D, generator=g, device=dev).half()
    k = torch.randn(B, Hk, S, D, generator=g, device=dev).half()
    v = torch.randn(B, Hk, S, D, generator=g, device=dev).half()

    def mean_ms(fn):
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.1:  # 0.1 s of calls, each waited for
            fn()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    ours_ms = mean_ms(lambda: flash_attn(q, k, v, True))
    res = {"shape": f"q [{B},{Hq},{S},{D}], k/v [{B},{Hk},{S},{D}] fp16, causal",
           "this_library_contiguous": {"ms": round(ours_ms, 4),
                                       "tflops": round(flops / ours_ms / 1e9, 1)}}
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            fn = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True,  # noqa: E731
                                                        enable_gqa=True)
            diff = (fn().float() - flash_attn(q, k, v, True).float()).abs().max().item()
            ms = mean_ms(fn)
        res["torch_sdpa_flash"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 1),
                                   "max_abs_diff_vs_this_library": diff,
                                   "library": f"torch {torch.__version__} SDPA flash backend"}
        res["speedup_over_torch_sdpa_flash"] = round(ms / ours_ms, 2)
    except RuntimeError as e:
        res["torch_sdpa_flash"] = {"unavailable": str(e)[:200]}
    del q, k, v
    # decode: one query row per sequence over contiguous K/V (the shape of the
    # contiguous-decode extra: B=8, 64/8 heads, 16384 keys), two rotating
    # caches so that every call reads HBM; GB/s of K/V plus q and o
    B, Hq, Hk, N = 8, 64, 8, 16384
    caches = [(torch.randn(B, Hk, N, D, generator=g, device=dev).half(),
               torch.randn(B, Hk, N, D, generator=g, device=dev).half()) for _ in range(2)]
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev).half()
    nbytes = B * Hk * N * D * 2 * 2 + 2 * B * Hq * D * 2
    it = [0]

    def rotating(fn):
        def call():
            kk, vv = caches[it[0] % 2]
            it[0] += 1
            return fn(kk, vv)
        return call

    ours_ms = mean_ms(rotating(lambda kk, vv: flash_attn(q, kk, vv, False)))
    dec = {"shape": f"q [{B},{Hq},1,{D}], k/v [{B},{Hk},{N},{D}] fp16, non-causal",
           "this_library_contiguous": {"ms": round(ours_ms, 4),
                                       "gbs": round(nbytes / ours_ms / 1e6, 1)}}
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            fn = lambda kk, vv: F.scaled_dot_product_attention(q, kk, vv, is_causal=False,  # noqa: E731
                                                               enable_gqa=True)
            diff = (fn(*caches[0]).float() - flash_attn(q, *caches[0], False).float()).abs().max().item()
            ms = mean_ms(rotating(fn))
        dec["torch_sdpa_flash"] = {"ms": round(ms, 4), "gbs": round(nbytes / ms / 1e6, 1),
                                   "max_abs_diff_vs_this_library": diff}
        dec["speedup_over_torch_sdpa_flash"] = round(ms / ours_ms, 2)
    except RuntimeError as e:
        dec["torch_sdpa_flash"] = {"unavailable": str(e)[:200]}
    res["decode"] = dec
    return res


def bench_cfg1(steps, warmup, dev):
    res = {}
    for dt in (torch.float16, torch.float32):
        q, k, v = workloads.cfg1(dev, dt)
        flops = workloads.causal_flops_contiguous(1, 8, 512, 512, 64)
        stream = torch.cuda.current_stream()

        def step(ev):
            if ev:
                ev[0].record(stream)
            flash_attn(q, k, v)
            if ev:
                ev[1].record(stream)

        wall, segs = timed(step, steps, warmup)
        mean_ms = statistics.fmean(s[0] for s in segs)
        res[str(dt).replace("torch.", "")] = {
            "kernel_ms": round(mean_ms, 4),
            "TFLOP/s": round(flops / (mean_ms * 1e-3) / 1e12, 3)}
    return res


def bench_token_major(steps, warmup, dev, traffic, H=40, KVH=8, Dh=128, t=32767, sets=3):
    """The INT8 engine's decode step (batch 1, token-major fp16 cache, fp32 q and
    out) at the Qwen-32B head counts and a 32K context, rotating `sets` caches
    (3 x 134 MB of K and V) so the step reads HBM, not the 256 MB MALL."""
    g = torch.Generator().manual_seed(1006)
    q = torch.randn(H, Dh, generator=g).to(dev)
    caches = []
    for _ in range(sets):
        k = torch.randn(t + 1, KVH, Dh, generator=g).to(torch.float16).to(dev)
        v = torch.randn(t + 1, KVH, Dh, generator=g).to(torch.float16).to(dev)
        caches.append((k, v))
    ws = torch.empty(token_major_workspace(H, KVH, Dh, t), dtype=torch.uint8, device=dev)
    nbytes = (t + 1) * KVH * Dh * 2 * 2 + 2 * H * Dh * 4
    stream = torch.cuda.current_stream()
    it = [0]

    def step(ev):
        k, v = caches[it[0] % sets]
        it[0] += 1
        if ev:
            ev[0].record(stream)
        decode_token_major(q, k, v, t, workspace=ws)
        if ev:
            ev[1].record(stream)

    _, mean_ms = back_to_back(step, steps, warmup)
    _, segs = timed(step, steps, 0)
    durs = [s[0] for s in segs]
    return {"kernel_ms_back_to_back": round(mean_ms, 4), "kernel_ms": dist(durs),
            "bytes_per_step": nbytes, "roofline": roofline("hbm", nbytes, mean_ms, traffic.get("decode_token_major")),
            "workload": {"heads": H, "kv_heads": KVH, "head_dim": Dh, "t": t,
                         "layout": "token-major [T, KVH, Dh] fp16, fp32 q/out"}}


def bench_contiguous_decode(steps, warmup, dev, B=8, Hq=64, Hk=8, N=16384, D=128, sets=2):
    """flash_attn over contiguous K/V [B, Hk, N, D] with few query rows (the
    reference serves every M with one launcher, csrc/flash_attn_sm75.cu:
    428-467): M = 1 (non-causal) and M = 4 (causal, the last four positions)
    at the Llama-70B head counts, on the split-K decode kernels. GB/s of the
    K/V bytes plus q and o, rotating `sets` caches (2 x 537 MB) so that every
    step reads HBM."""
    g = torch.Generator(device=dev)
    g.manual_seed(1008)
    caches = [(torch.randn(B, Hk, N, D, generator=g, device=dev).half(),
               torch.randn(B, Hk, N, D, generator=g, device=dev).half()) for _ in range(sets)]
    out = {}
    for M, causal in ((1, False), (4, True)):
        q = torch.randn(B, Hq, M, D, generator=g, device=dev).half()
        qo = N - M
        nbytes = B * Hk * N * D * 2 * 2 + 2 * B * Hq * M * D * 2
        it = [0]

        def step(ev):
            k, v = caches[it[0] % sets]
            it[0] += 1
            if ev:
                ev[0].record()
            flash_attn(q, k, v, causal, qo, 0)
            if ev:
                ev[1].record()

        _, mean_ms = back_to_back(step, steps, warmup)
        out[f"M{M}"] = {"kernel_ms_back_to_back": round(mean_ms, 4), "bytes_per_step": nbytes,
                        "roofline": roofline("hbm", nbytes, mean_ms),
                        "causal": causal, "q_offset": qo}
    out["workload"] = {"B": B, "Hq": Hq, "Hk": Hk, "N": N, "D": D,
                       "path": "fa_flash_attn_fwd_ws: split-K decode kernels + combine"}
    return out


# ------------------------------------------------------------ CPU baseline ---

def cpu_threads():
    """Host threads for the CPU baseline: the CPUs this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS when it is set. A one-GPU
    job on the benchmark box is allotted a share of the host (16 CPUs,
    OMP_NUM_THREADS=16) although os.cpu_count() reports every core of the
    machine; more threads than the share would oversubscribe it."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        avail = min(avail, int(omp))
    return max(1, avail)


def cpu_baseline_paged(w, kind, budget_s=10.0):
    """Time the oracle's restatement of the reference CPU path on this host.

    The sample spreads over the workload's sequence lengths: up to
    `n_seq` sequences at evenly spaced ranks of their key counts (shortest to
    longest), each timed on a prefix of its q heads sized from a probe so that
    the whole sample takes about `budget_s`. Each sampled sequence gives a
    rate (its algorithmic work over its time); every sequence of the workload
    is then charged its own work at the rate of the sampled sequence nearest
    in key count, and the reported value is the whole job's work over that
    extrapolated time (same unit as the GPU figure). Attention only: the
    append of the decode step is a copy of B rows."""
    from oracle import attention as ora

    threads = cpu_threads()
    torch.set_num_threads(threads)
    threads = torch.get_num_threads()
    q = w.q.cpu()
    kp, vp = w.k_pool.cpu(), w.v_pool.cpu()
    bt = w.block_table.cpu()
    sl = w.seqlen.cpu()
    hm = w.head_map.cpu()
    qo = w.q_offsets.cpu() if w.q_offsets is not None else 0

    def pairs_of(b):
        n = w.lengths[b]
        if not w.causal:
            return w.M * n
        off = w.q_offsets_host[b] if w.q_offsets_host else 0
        return sum(max(0, min(n, off + i + 1)) for i in range(w.M))

    def work_of(b, nh):
        if kind == "flops":
            return 4.0 * w.D * pairs_of(b) * nh
        return w.lengths[b] * w.Hk * w.D * 2 * 2 * nh / w.Hq + 2 * nh * w.M * w.D * 2

    def run(b, nh):
        ora.cpu_flash_attn_paged(q, kp, vp, sl, 16, hm, w.causal, qo, 0, block_table=bt,
                                 batches=[b], heads=list(range(nh)))

    order = sorted(range(w.B), key=lambda b: (pairs_of(b), b))
    n_seq = min(w.B, 4 if w.B <= 16 else 6)
    picks = sorted({order[min(w.B - 1, int((i + 0.5) * w.B / n_seq))] for i in range(n_seq)},
                   key=lambda b: pairs_of(b))
    run(picks[0], 1)                   # warm-up
    t0 = time.perf_counter()
    run(picks[0], 1)
    per_pair = max(time.perf_counter() - t0, 1e-5) / max(pairs_of(picks[0]), 1)
    share = budget_s / len(picks)
    rates, plan, spent = {}, [], 0.0
    for b in picks:
        nh = max(1, min(w.Hq, int(share / max(per_pair * max(pairs_of(b), 1), 1e-9))))
        # repeated while the sequence's share of the budget lasts (at least
        # once), so that short sequences are not timed on a few milliseconds
        reps, t0 = 0, time.perf_counter()
        while True:
            run(b, nh)
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= 0.5 * share or reps >= 1000:
                break
        spent += dt
        rates[b] = work_of(b, nh) * reps / max(dt, 1e-9)
        plan.append((b, nh, reps, dt))
    # every sequence at the rate of the sampled one nearest in key count
    job_work, job_time = 0.0, 0.0
    for b in range(w.B):
        near = min(picks, key=lambda c: (abs(pairs_of(c) - pairs_of(b)), c))
        wb = work_of(b, w.Hq)
        job_work += wb
        job_time += wb / rates[near]
    scale = 1e12 if kind == "flops" else 1e9
    value, unit = job_work / job_time / scale, ("TFLOP/s" if kind == "flops" else "GB/s")
    heads_done = sum(nh for _, nh, _, _ in plan)
    sample = (f"{heads_done} of {w.B * w.Hq} (sequence, head) pairs from {len(picks)} of {w.B} "
              "sequences spread over the key counts ("
              + ", ".join(f"seq {b}: {w.lengths[b]} keys, {nh} heads x {reps}, {dt:.2f} s"
                          for b, nh, reps, dt in plan)
              + f"); {spent:.2f} s on the host; the whole job extrapolated at each sampled "
              "sequence's rate to the sequences nearest in key count")
    return {"value": round(value, 4), "unit": unit, "cores": threads, "kind": "port",
            "sample": sample, "extrapolated": heads_done < w.B * w.Hq,
            "cpu_count": os.cpu_count(), "threads_note": "torch intra-op threads = the CPUs "
            "this process may use (affinity, capped by OMP_NUM_THREADS); cpu_count is the "
            "whole machine", "cpu": cpu_info(), "torch": torch.__version__}


# -------------------------------------------------------------------- main ---

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="2,4,3,5,5r,1,tm,gemm")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy a MIB-mebibyte device buffer --steps times (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        dev = torch.device("cuda", 0)
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": args.steps}))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py measures one GPU: this attention path runs on a "
                                   "single MI355X (no sharding, no collectives); use --gpus 1"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda", 0)
    cfgs = [c.strip() for c in args.configs.split(",") if c.strip()]
    traffic = load_traffic()
    K, W = args.steps, args.warmup
    result = {}
    extra = {}
    cpu = {}

    if "2" in cfgs:
        log("cfg2: building workload")
        w2 = workloads.cfg2(dev)
        result = bench_prefill(w2, K, W, "prefill_cfg2", traffic)
        log(f"cfg2: {result['value']} TFLOP/s, kernel {result['kernel_ms']['mean']} ms")
        if not args.no_cpu_baseline:
            cpu["cfg2"] = cpu_baseline_paged(w2, "flops")
            log(f"cfg2 cpu: {cpu['cfg2']}")
        del w2
    if "4" in cfgs:
        log("cfg4: building workload")
        w4 = workloads.cfg4(dev)
        extra["decode_cfg4"] = bench_decode(w4, K, W, "decode_cfg4", traffic)
        log(f"cfg4: decode {extra['decode_cfg4']['roofline']['achieved']} GB/s")
        rope = build_rope_cache(max(w4.lengths) + 1, w4.D, device=dev)
        extra["decode_cfg4_rope"] = bench_decode(w4, K, W, "decode_cfg4", traffic, rope=rope)
        log(f"cfg4 with fused rotary embedding: decode "
            f"{extra['decode_cfg4_rope']['roofline']['achieved']} GB/s")
        extra["decode_cfg4_fused_append"] = bench_decode_fused(w4, K, W, extra["decode_cfg4"])
        log(f"cfg4 fused append + decode: {extra['decode_cfg4_fused_append']['step_ms_back_to_back']}"
            f" ms per step against {extra['decode_cfg4']['end_to_end_ms']} ms as two calls")
        extra["decode_cfg4_fused_append_rope"] = bench_decode_fused(
            w4, K, W, extra["decode_cfg4_rope"], rope=rope)
        extra["decode_cfg4_query_rows"] = bench_decode_rows(w4, K, W)
        log("cfg4 pool with M query rows: " + ", ".join(
            f"{k} {v['roofline']['achieved']} GB/s ({v['path']})"
            for k, v in extra["decode_cfg4_query_rows"].items()))
        if not args.no_cpu_baseline:
            cpu["cfg4"] = cpu_baseline_paged(w4, "bytes")
            log(f"cfg4 cpu: {cpu['cfg4']}")
        del w4, rope
    if "3" in cfgs:
        log("cfg3: building workload (two pools)")
        w3 = workloads.cfg3(dev)
        w3b = workloads.cfg3(dev)
        extra["decode_cfg3"] = bench_decode(w3, K, W, "decode_cfg3", traffic, rotate=w3b)
        log(f"cfg3: decode {extra['decode_cfg3']['roofline']['achieved']} GB/s")
        if not args.no_cpu_baseline:
            cpu["cfg3"] = cpu_baseline_paged(w3, "bytes")
        del w3, w3b
    if "5" in cfgs:
        log("cfg5: building workload")
        w5 = workloads.cfg5(dev)
        extra["chunked_prefill_cfg5"] = bench_prefill(w5, max(3, K // 4), min(W, 2),
                                                      "prefill_cfg5", traffic)
        log(f"cfg5: {extra['chunked_prefill_cfg5']['value']} TFLOP/s")
        if not args.no_cpu_baseline:
            cpu["cfg5"] = cpu_baseline_paged(w5, "flops")
        del w5
    if "5r" in cfgs:
        log("cfg5 ragged: building workload")
        w5r = workloads.cfg5_ragged(dev)
        ks = max(3, K // 4)
        packed = bench_prefill(w5r, ks, min(W, 2), "prefill_cfg5_ragged", traffic, q_lens=w5r.q_lens)
        padded = bench_prefill(w5r, ks, min(W, 2), "prefill_cfg5_ragged_padded", traffic)
        extra["chunked_prefill_cfg5_ragged"] = {
            "note": "ragged chunks (live rows U[64, 512] of 512): TFLOP/s of the live rows' "
                    "algorithmic flops, with q_lens (padding rows skipped) and without "
                    "(padding rows computed)",
            "packed_q_lens": packed, "padded": padded,
            "speedup": round(padded["kernel_ms_back_to_back"] / packed["kernel_ms_back_to_back"], 3)}
        log(f"cfg5 ragged: packed {packed['value']} TFLOP/s, padded {padded['value']} TFLOP/s")
        del w5r
    if "1" in cfgs:
        extra["cfg1_contiguous"] = bench_cfg1(K, W, dev)
        extra["contiguous_decode"] = bench_contiguous_decode(K, W, dev)
        log("contiguous decode: " + ", ".join(
            f"{k} {v['roofline']['achieved']} GB/s" for k, v in extra["contiguous_decode"].items()
            if k.startswith("M")))
    if "tm" in cfgs:
        extra["int8_engine_decode_token_major"] = bench_token_major(K, W, dev, traffic)
        log(f"token-major decode: "
            f"{extra['int8_engine_decode_token_major']['roofline']['achieved']} GB/s")
    # The vendor references run last. Measured right after them, the
    # token-major step took 34.9 us against 31.6 us before them (full bench
    # runs on one box).
    if "gemm" in cfgs:
        extra["fp16_gemm_reference"] = bench_gemm_reference(dev)
        log(f"fp16 GEMM reference: {extra['fp16_gemm_reference']['tflops']} TFLOP/s")
        try:  # a context figure only: a torch without this backend must not end the run
            extra["vendor_flash_attention_reference"] = bench_vendor_attention_reference(dev)
        except Exception as e:  # noqa: BLE001
            extra["vendor_flash_attention_reference"] = {"unavailable": f"{type(e).__name__}: {e}"[:200]}
        log(f"vendor flash attention reference: {extra['vendor_flash_attention_reference']}")
    torch.cuda.synchronize()

    if not result:  # prefill not requested: report the first measured config as headline
        key = next((k for k, v in extra.items() if "value" in v), None)
        if key is not None:
            result = extra.pop(key)
        else:
            key = next((k for k, v in extra.items() if "roofline" in v), None)
            if key is None:
                # entries that hold several measured cases (contiguous decode
                # M1 / M4): the first of them
                for k, v in extra.items():
                    sub = next((s for s in v.values() if isinstance(s, dict) and "roofline" in s),
                               None) if isinstance(v, dict) else None
                    if sub is not None:
                        key = k
                        extra[k] = dict(sub, kernel_ms={"mean": sub.get("kernel_ms_back_to_back")},
                                        cases=v)
                        break
            if key is None:
                print(json.dumps({"error": "no attention configuration requested", "extra": extra}))
                sys.exit(2)
            result = dict(extra.pop(key))
            result["value"] = result["roofline"]["achieved"]
            result["unit"] = result["roofline"]["unit"]
            result["ms_per_step"] = result["kernel_ms"]["mean"]
    decode = extra.pop("decode_cfg4", None)
    line = {
        "metric": METRIC,
        "value": result["value"],
        "unit": result["unit"],
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": result["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) Q/K/V, random block tables)",
        "config": {"workload": "cfg2_prefill_qwen32b" if "2" in cfgs else "custom",
                   **result.get("workload", {})},
        "roofline": result["roofline"],
        "traffic_source": {"file": "profiles/traffic.json",
                           "measured_at": traffic.get("_measured_at"),
                           "how": "constant from rocprofv3 --pmc FETCH_SIZE x 2 + WRITE_SIZE "
                                  "per dispatch (scaled by a 1 GiB copy), not measured in "
                                  "this run"},
        "cpu_baseline": cpu.get("cfg2"),
        "kernel_ms_back_to_back": result.get("kernel_ms_back_to_back"),
        "kernel_ms": result.get("kernel_ms"),
    }
    if "cases" in result:  # a headline taken from an entry of several cases
        line["cases"] = result["cases"]
    if decode is not None:
        decode["cpu_baseline"] = cpu.get("cfg4")
        line["decode"] = decode
    for k, v in extra.items():
        cfg_key = {"decode_cfg3": "cfg3", "chunked_prefill_cfg5": "cfg5"}.get(k)
        if isinstance(v, dict) and cfg_key and cfg_key in cpu:
            v["cpu_baseline"] = cpu[cfg_key]
    line["extra"] = extra
    line["device"] = torch.cuda.get_device_name(0)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
