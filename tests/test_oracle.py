"""CPU tests that pin the oracle (no GPU).

* The restatement of the reference's CPU math path (oracle.attention.cpu_*)
  is checked bit-for-bit against golden vectors the reference's own ops.py
  produced (tests/golden/make_golden.py).
* The fp64 closed form is checked against a brute-force loop, against torch's
  SDPA in float64, and against invariants the mathematics fixes; mutated
  variants (a plausible bug planted in a copy of the oracle) must fail them.
* The page-map helpers are checked against the reference's flatten and
  append known-answer test (flash_tests/test_append_fast.py:16-38).
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as ora

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_cpu_path.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def _bitexact(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a, b, equal_nan=True)


# ---------------------------------------------------------------- golden ----

ATTN_CASES = ["attn_f16_causal", "attn_f16_offset", "attn_f32_causal", "attn_f32_noncausal",
              "attn_f16_kofs"]
PAGED_CASES = ["paged_prefill", "paged_decode", "paged_decode_mha"]


@pytest.mark.parametrize("name", ATTN_CASES)
def test_cpu_flash_attn_bitexact_vs_reference(golden, name):
    causal, qo, ko = golden[f"{name}/meta"].tolist()
    o = ora.cpu_flash_attn(_t(golden[f"{name}/q"]), _t(golden[f"{name}/k"]),
                           _t(golden[f"{name}/v"]), bool(causal), qo, ko)
    assert _bitexact(o.numpy(), golden[f"{name}/o"])


@pytest.mark.parametrize("name", PAGED_CASES)
def test_cpu_flash_attn_paged_bitexact_vs_reference(golden, name):
    causal, qo, ko, ps = golden[f"{name}/meta"].tolist()
    g = lambda k: _t(golden[f"{name}/{k}"])  # noqa: E731
    o = ora.cpu_flash_attn_paged(g("q"), g("k_pages"), g("v_pages"), g("seqlen"), ps,
                                 g("head_map"), bool(causal), qo, ko)
    assert _bitexact(o.numpy(), golden[f"{name}/o"])


def test_cpu_paged_kv_append_bitexact_vs_reference(golden):
    start, ps = golden["append/meta"].tolist()
    kp = _t(golden["append/k_pages_in"]).clone()
    vp = _t(golden["append/v_pages_in"]).clone()
    ora.cpu_paged_kv_append(kp, vp, _t(golden["append/k_new"]), _t(golden["append/v_new"]),
                            start, ps)
    assert _bitexact(kp.numpy(), golden["append/k_pages_out"])
    assert _bitexact(vp.numpy(), golden["append/v_pages_out"])
    ko, vo = ora.append_f16(golden["append/k_pages_in"], golden["append/v_pages_in"],
                            golden["append/k_new"], golden["append/v_new"], start, ps)
    assert _bitexact(ko, golden["append/k_pages_out"])
    assert _bitexact(vo, golden["append/v_pages_out"])


@pytest.mark.parametrize("name", ATTN_CASES)
def test_reference_cpu_path_within_tolerance_of_f64(golden, name):
    causal, qo, ko = golden[f"{name}/meta"].tolist()
    ref = ora.attention_f64(golden[f"{name}/q"], golden[f"{name}/k"], golden[f"{name}/v"],
                            bool(causal), qo, ko)
    ok, worst = ora.within_tolerance(golden[f"{name}/o"], ref)
    assert ok, worst


@pytest.mark.parametrize("name", PAGED_CASES)
def test_reference_paged_within_tolerance_of_f64(golden, name):
    causal, qo, ko, ps = golden[f"{name}/meta"].tolist()
    g = lambda k: golden[f"{name}/{k}"]  # noqa: E731
    B = g("q").shape[0]
    k = ora.gather_kv(g("k_pages"), B, ps)
    v = ora.gather_kv(g("v_pages"), B, ps)
    ref = ora.attention_f64(g("q"), k, v, bool(causal), qo, ko, kv_len=g("seqlen"),
                            head_map=g("head_map"))
    ok, worst = ora.within_tolerance(g("o"), ref)
    assert ok, worst


# ------------------------------------------------------------ fp64 form ----

def brute_force(q, k, v, causal, qo, ko, kv_len=None, head_map=None):
    """Independent scalar loops (tiny shapes only)."""
    B, Hq, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    out = np.zeros((B, Hq, M, D))
    for b in range(B):
        n = N if kv_len is None else int(kv_len[b])
        for h in range(Hq):
            hk = h // (Hq // Hk) if head_map is None else int(head_map[h])
            for i in range(M):
                vis = [j for j in range(n) if (not causal) or (ko + j <= qo + i)]
                if n == 0:
                    continue
                if not vis:
                    out[b, h, i] = np.nan
                    continue
                sc = [sum(float(q[b, h, i, d]) * float(k[b, hk, j, d]) for d in range(D))
                      / math.sqrt(D) for j in vis]
                mx = max(sc)
                w = [math.exp(s - mx) for s in sc]
                tot = sum(w)
                for d in range(D):
                    out[b, h, i, d] = sum(wj * float(v[b, hk, j, d]) for wj, j in zip(w, vis)) / tot
    return out


def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float64)


@pytest.mark.parametrize("causal,qo,ko", [(True, 0, 0), (True, 3, 1), (False, 0, 0), (True, 0, 4)])
def test_attention_f64_matches_brute_force(causal, qo, ko):
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 2, 4, 5, 8), _rand(rng, 2, 2, 7, 8), _rand(rng, 2, 2, 7, 8)
    kv_len = [7, 5]
    ref = ora.attention_f64(q, k, v, causal, qo, ko, kv_len=kv_len)
    bf = brute_force(q, k, v, causal, qo, ko, kv_len=kv_len)
    np.testing.assert_allclose(ref, bf, rtol=1e-12, atol=1e-12, equal_nan=True)


def test_attention_f64_matches_torch_sdpa():
    rng = np.random.default_rng(2)
    B, Hq, Hk, M, N, D = 2, 6, 2, 9, 13, 16
    q, k, v = _rand(rng, B, Hq, M, D), _rand(rng, B, Hk, N, D), _rand(rng, B, Hk, N, D)
    qo, ko = 4, 0
    ref = ora.attention_f64(q, k, v, True, qo, ko)
    kr = torch.from_numpy(k).repeat_interleave(Hq // Hk, dim=1)
    vr = torch.from_numpy(v).repeat_interleave(Hq // Hk, dim=1)
    mask = (torch.arange(N)[None, :] + ko) <= (torch.arange(M)[:, None] + qo)
    sd = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), kr, vr,
                                                          attn_mask=mask)
    np.testing.assert_allclose(ref, sd.numpy(), rtol=1e-10, atol=1e-10)


def test_attention_f64_invariants():
    rng = np.random.default_rng(3)
    B, H, M, N, D = 1, 2, 6, 6, 8
    q, k, v = _rand(rng, B, H, M, D), _rand(rng, B, H, N, D), _rand(rng, B, H, N, D)
    out = ora.attention_f64(q, k, v, True)
    # causal row 0 sees only key 0
    np.testing.assert_allclose(out[:, :, 0], v[:, :, 0], rtol=0, atol=1e-12)
    # zero queries -> equal scores -> mean of the visible V rows
    z = ora.attention_f64(np.zeros_like(q), k, v, True)
    for i in range(M):
        np.testing.assert_allclose(z[0, :, i], v[0, :, : i + 1].mean(axis=1), atol=1e-12)
    # key permutation invariance (non-causal)
    perm = rng.permutation(N)
    a = ora.attention_f64(q, k, v, False)
    b = ora.attention_f64(q, k[:, :, perm], v[:, :, perm], False)
    np.testing.assert_allclose(a, b, atol=1e-12)
    # decode: non-causal == causal with q_offset >= kv_len - 1
    q1 = q[:, :, :1]
    np.testing.assert_allclose(ora.attention_f64(q1, k, v, False),
                               ora.attention_f64(q1, k, v, True, q_offset=N - 1), atol=1e-12)
    # fully masked row -> NaN; zero keys -> 0 (reference CPU path semantics)
    m = ora.attention_f64(q, k, v, True, q_offset=0, k_offset=2)
    assert np.isnan(m[:, :, :2]).all() and not np.isnan(m[:, :, 2:]).any()
    e = ora.attention_f64(q, k, v, True, kv_len=[0])
    assert (e == 0).all()


def test_attention_f64_gqa_equals_repeated_mha():
    rng = np.random.default_rng(4)
    q, k, v = _rand(rng, 1, 8, 5, 8), _rand(rng, 1, 2, 9, 8), _rand(rng, 1, 2, 9, 8)
    g = ora.attention_f64(q, k, v, True, q_offset=4)
    m = ora.attention_f64(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), True, q_offset=4)
    np.testing.assert_allclose(g, m, atol=1e-12)
    hm = np.array([1, 0, 1, 0, 1, 0, 1, 0])
    g2 = ora.attention_f64(q, k, v, False, head_map=hm)
    m2 = ora.attention_f64(q, k[:, hm], v[:, hm], False)
    np.testing.assert_allclose(g2, m2, atol=1e-12)


def _planted(kind):
    """Copies of the oracle with one plausible bug each."""
    def f(q, k, v, causal, qo, ko, kv_len=None):
        if kind == "no_scale":
            return ora.attention_f64(q * math.sqrt(q.shape[-1]), k, v, causal, qo, ko, kv_len)
        if kind == "swap_kv":
            return ora.attention_f64(q, v, k, causal, qo, ko, kv_len)
        if kind == "causal_off_by_one":
            return ora.attention_f64(q, k, v, causal, qo + 1, ko, kv_len)
        if kind == "ignore_kv_len":
            return ora.attention_f64(q, k, v, causal, qo, ko, None)
        raise ValueError(kind)
    return f


@pytest.mark.parametrize("kind", ["no_scale", "swap_kv", "causal_off_by_one", "ignore_kv_len"])
def test_planted_oracle_bugs_are_caught(kind):
    rng = np.random.default_rng(5)
    q, k, v = _rand(rng, 1, 2, 4, 8), _rand(rng, 1, 2, 6, 8), _rand(rng, 1, 2, 6, 8)
    kv_len = [3]  # below the causal limit of the last rows, so it matters
    bf = brute_force(q, k, v, True, 1, 0, kv_len=kv_len)
    bad = _planted(kind)(q, k, v, True, 1, 0, kv_len)
    ok, _ = ora.within_tolerance(bad, bf)
    assert not ok


# ------------------------------------------------------------ page maps ----

def test_gather_identity_matches_reference_flatten():
    rng = np.random.default_rng(6)
    B, Hk, P, PS, D = 2, 3, 4, 16, 8
    kp = rng.standard_normal((B, Hk, P, PS, D)).astype(np.float16)
    flat = ora.gather_kv(kp, B, PS)
    np.testing.assert_array_equal(flat, kp.reshape(B, Hk, P * PS, D))


def test_gather_block_table_recovers_unpermuted_pool():
    rng = np.random.default_rng(7)
    B, Hk, P, PS, D = 3, 2, 5, 16, 8
    seq = rng.standard_normal((B, Hk, P, PS, D)).astype(np.float16)
    perm = rng.permutation(B * P)                 # logical (b, p) -> physical id
    pool = np.zeros((1, Hk, B * P, PS, D), np.float16)
    bt = perm.reshape(B, P).astype(np.int32)
    for b in range(B):
        for p in range(P):
            pool[0, :, bt[b, p]] = seq[b, :, p]
    got = ora.gather_kv(pool, B, PS, block_table=bt)
    np.testing.assert_array_equal(got, seq.reshape(B, Hk, P * PS, D))


def test_append_kat_shape_matches_elementwise_loop():
    # flash_tests/test_append_fast.py:16-38: B=2, Hk=4, P=8, PS=128, D=128, T=96, start=145
    rng = np.random.default_rng(8)
    B, Hk, P, PS, D, T, start = 2, 4, 8, 128, 128, 96, 145
    kp = np.zeros((B, Hk, P, PS, D), np.float16)
    vp = np.zeros_like(kp)
    kn = rng.standard_normal((B, Hk, T, D)).astype(np.float16)
    vn = rng.standard_normal((B, Hk, T, D)).astype(np.float16)
    ko, vo = ora.append_f16(kp, vp, kn, vn, start, PS)
    ke, ve = kp.copy(), vp.copy()
    for t in range(T):
        pos = start + t
        ke[:, :, pos // PS, pos - (pos // PS) * PS, :] = kn[:, :, t, :]
        ve[:, :, pos // PS, pos - (pos // PS) * PS, :] = vn[:, :, t, :]
    assert _bitexact(ko, ke) and _bitexact(vo, ve)
    assert ko[:, :, 1, 17].tobytes() == kn[:, :, 0].tobytes()     # page-crossing start


def test_append_skips_out_of_range_and_block_table():
    rng = np.random.default_rng(9)
    B, Hk, P, PS, D, T = 2, 1, 2, 4, 8, 3
    kp = np.zeros((B, Hk, P, PS, D), np.float16)
    kn = rng.standard_normal((B, Hk, T, D)).astype(np.float16)
    ko, _ = ora.append_f16(kp, kp, kn, kn, [6, -2], PS)  # b0 crosses capacity 8; b1 negative
    assert _bitexact(ko[0, :, 1, 2], kn[0, :, 0]) and _bitexact(ko[0, :, 1, 3], kn[0, :, 1])
    assert _bitexact(ko[1, :, 0, 0], kn[1, :, 2]) and np.count_nonzero(ko[1]) == D - np.sum(kn[1, :, 2] == 0)
    bt = np.array([[3, 2], [1, -1]], np.int32)
    pool = np.zeros((1, Hk, 4, PS, D), np.float16)
    po, _ = ora.append_f16(pool, pool, kn, kn, [1, 3], PS, block_table=bt)
    assert _bitexact(po[0, :, 3, 1], kn[0, :, 0]) and _bitexact(po[0, :, 1, 3], kn[1, :, 0])
    assert not po[0, :, 0].any()  # b1 tokens 1..2 fall on the unmapped page -> skipped


# ------------------------------------------------------------- rotary ----

def test_rope_tables_match_closed_form():
    cos, sin = ora.rope_tables(300, 128)
    half = 64
    ang = np.arange(300)[:, None] * (10000.0 ** (-np.arange(half) / half))[None, :]
    assert cos.shape == (300, 64) and cos.dtype == np.float16
    assert np.allclose(cos.astype(np.float64), np.cos(ang), atol=1e-3, rtol=0)
    assert np.allclose(sin.astype(np.float64), np.sin(ang), atol=1e-3, rtol=0)


def test_rope_f16_bitexact_vs_torch_fp16_arithmetic():
    """The oracle's numpy emulation equals torch's fp16 CPU ops on the same
    half-split expression, bit for bit."""
    g = torch.Generator().manual_seed(5)
    for D in (64, 128):
        cos, sin = ora.rope_tables(512, D)
        x = (torch.randn(2, 3, 40, D, generator=g) * 4).to(torch.float16)
        pos = torch.randint(0, 512, (40,), generator=g)
        c = torch.from_numpy(cos)[pos].view(1, 1, 40, D // 2)
        s = torch.from_numpy(sin)[pos].view(1, 1, 40, D // 2)
        x1, x2 = x[..., :D // 2], x[..., D // 2:]
        want = torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1).numpy()
        got = ora.rope_f16(x, cos, sin, pos.numpy())
        assert got.dtype == np.float16 and np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_rope_f16_invariants():
    cos, sin = ora.rope_tables(4096, 128)
    g = np.random.default_rng(3)
    x = g.standard_normal((1, 2, 8, 128)).astype(np.float16)
    # position 0: cos = 1, sin = 0 -> identity
    assert np.array_equal(ora.rope_f16(x, cos, sin, np.zeros(8, np.int64)), x)
    # rotation keeps the norm of every (x1_j, x2_j) pair (to fp16 rounding)
    pos = g.integers(0, 4096, 8)
    y = ora.rope_f16(x, cos, sin, pos).astype(np.float64)
    xn = np.hypot(x[..., :64].astype(np.float64), x[..., 64:].astype(np.float64))
    yn = np.hypot(y[..., :64], y[..., 64:])
    assert np.allclose(xn, yn, atol=2e-2, rtol=4e-3)
    # rotating by p1 then p2 equals rotating by p1 + p2 (angles add)
    p1, p2 = g.integers(0, 2000, 8), g.integers(0, 2000, 8)
    a = ora.rope_f16(ora.rope_f16(x, cos, sin, p1), cos, sin, p2).astype(np.float64)
    b = ora.rope_f16(x, cos, sin, p1 + p2).astype(np.float64)
    assert np.allclose(a, b, atol=3e-2, rtol=1e-2)


def test_rope_planted_sign_error_is_caught():
    cos, sin = ora.rope_tables(4096, 64)
    g = np.random.default_rng(4)
    x = g.standard_normal((1, 1, 16, 64)).astype(np.float16)
    p1, p2 = g.integers(1, 2000, 16), g.integers(1, 2000, 16)

    def wrong(v, pos):  # y1 = x1*c + x2*s (sign flipped)
        c, s = cos[pos].astype(np.float32), sin[pos].astype(np.float32)
        v1, v2 = v[..., :32].astype(np.float32), v[..., 32:].astype(np.float32)
        return np.concatenate([(v1 * c + v2 * s), (v1 * s + v2 * c)], -1).astype(np.float16)

    a = wrong(wrong(x, p1), p2).astype(np.float64)
    b = wrong(x, p1 + p2).astype(np.float64)
    assert not np.allclose(a, b, atol=3e-2, rtol=1e-2)


def test_package_rope_tables_match_the_oracle_tables():
    """hrm_flashrenderer_amd.build_rope_cache (the product's table builder)
    against the oracle's restatement of engine/rope.py:6-13 (fp16 rounding of
    the same fp32 angles; at most one fp16 ulp apart where cos/sin differ in
    the last bit of their fp32 evaluation)."""
    from hrm_flashrenderer_amd.rope import build_rope_cache
    for D in (64, 128):
        c, s = build_rope_cache(1000, D, device="cpu")
        oc, os_ = ora.rope_tables(1000, D)
        assert c.shape == (1000, D // 2) and c.dtype == torch.float16
        dc = np.abs(c.numpy().astype(np.float64) - oc.astype(np.float64))
        ds = np.abs(s.numpy().astype(np.float64) - os_.astype(np.float64))
        assert dc.max() <= 2 ** -11 and ds.max() <= 2 ** -11


# ---- the INT8 engine's token-major decode (deepseek_native_engine.sh:562-604) ----

def _engine_cache(T, KVH, Dh, H, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, Dh, generator=g, dtype=torch.float32)
    k = torch.randn(T, KVH, Dh, generator=g).to(torch.float16)
    v = torch.randn(T, KVH, Dh, generator=g).to(torch.float16)
    return q, k, v


def test_token_major_decode_equals_closed_form_with_modulo_heads():
    H, KVH, Dh, T, t = 10, 4, 16, 40, 23
    q, k, v = _engine_cache(T, KVH, Dh, H, 5)
    out = ora.decode_token_major_f64(q, k, v, t)
    # the same attention through attention_f64: [1, KVH, t+1, Dh] and head map h % KVH
    kk = k[:t + 1].permute(1, 0, 2)[None]
    vv = v[:t + 1].permute(1, 0, 2)[None]
    ref = ora.attention_f64(q[None, :, None, :], kk, vv, False,
                            head_map=[h % KVH for h in range(H)])[0, :, 0]
    assert np.allclose(out, ref, rtol=0, atol=1e-12)


def test_token_major_decode_matches_the_engine_recurrence():
    # per-key online softmax exactly as attn_decode updates (m, s, acc), :571-600
    H, KVH, Dh, T, t = 6, 2, 8, 9, 6
    q, k, v = _engine_cache(T, KVH, Dh, H, 6)
    out = ora.decode_token_major_f64(q, k, v, t, scale=1 / math.sqrt(Dh))
    for h in range(H):
        kvh = h % KVH
        m, s, acc = -1e30, 0.0, np.zeros(Dh)
        for kpos in range(t + 1):
            dot = float(np.dot(q[h].double().numpy(), k[kpos, kvh].double().numpy())) / math.sqrt(Dh)
            new_m = max(m, dot)
            e_old, e_new = math.exp(m - new_m), math.exp(dot - new_m)
            acc = acc * e_old + v[kpos, kvh].double().numpy() * e_new
            s = s * e_old + e_new
            m = new_m
        assert np.allclose(out[h], acc / max(s, 1e-10), rtol=0, atol=1e-12)


def test_token_major_decode_invariants_and_planted_head_map():
    H, KVH, Dh, T = 8, 2, 16, 12
    q, k, v = _engine_cache(T, KVH, Dh, H, 7)
    out0 = ora.decode_token_major_f64(q, k, v, 0)   # one visible key -> its value row
    for h in range(H):
        assert np.allclose(out0[h], v[0, h % KVH].double().numpy(), atol=1e-12)
    out = ora.decode_token_major_f64(q, k, v, T - 1)
    planted = ora.decode_token_major_f64(q, k, v, T - 1, head_map=[h // (H // KVH) for h in range(H)])
    assert not np.allclose(out, planted, atol=1e-3)
    # keys past t never matter
    k2, v2 = k.clone(), v.clone()
    k2[6:] = float("nan")
    v2[6:] = float("nan")
    assert np.array_equal(ora.decode_token_major_f64(q, k2, v2, 5), ora.decode_token_major_f64(q, k, v, 5))
