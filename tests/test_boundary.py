"""CPU tests of the drop-in boundary (no GPU needed).

* libfa_mi355x.so loads and exports every function include/fa_mi355x.h declares.
* The C ABI rejects bad arguments with status codes and the reference's
  messages before touching the device.
* The Python API keeps the reference's names, positional order and defaults
  (flashattention_custom/ops.py:79-99) and raises the reference extension's
  messages (csrc/ext.cpp:31-87) for bad arguments.
* The custom ops are registered with shape-only (fake) implementations.
"""
import ctypes
import inspect
import os
import re

import pytest
import torch

from hrm_flashrenderer_amd import _lib, ops

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fa_mi355x.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted([
        "fa_abi_version", "fa_decode_token_major", "fa_decode_token_major_workspace_bytes",
        "fa_flash_attn_fwd", "fa_flash_attn_fwd_ws", "fa_flash_attn_workspace_bytes",
        "fa_flash_attn_paged_append_fwd", "fa_flash_attn_paged_fwd",
        "fa_flash_attn_paged_fwd_noalloc",
        "fa_flash_attn_paged_rope_fwd", "fa_last_error", "fa_paged_kv_append",
        "fa_paged_kv_append_rope", "fa_paged_kv_scatter", "fa_paged_workspace_bytes"])


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert {s[0] for s in _lib.SYMBOLS} == set(declared_functions())
    assert lib.fa_abi_version() == _lib.FA_ABI_VERSION


def _status_and_message(rc):
    return rc, _lib.load().fa_last_error().decode()


def test_fused_append_entry_rejects_bad_arguments_without_a_device():
    """fa_flash_attn_paged_append_fwd validates before it launches anything."""
    lib = _lib.load()
    P = ctypes.c_void_p(16)  # never dereferenced: validation fails first

    def call(advance=1, start_pos=0, start_positions=None, cos=None, sin=None, rope_len=0, D=128,
             NB=2, page_size=16):
        return _status_and_message(lib.fa_flash_attn_paged_append_fwd(
            P, P, P, P, page_size, P, P, 2, 8, 1, D, NB, 2, 4, 0, 0, None, None, 0, 4, P, P,
            advance, start_pos, start_positions, cos, sin, rope_len, None, 0, None))

    assert call(advance=2) == (-1, "advance must be 0 or 1")
    assert call(advance=1, start_pos=3) == (
        -1, "with advance the positions are the lengths: no start positions")
    assert call(advance=1, start_positions=P) == (
        -1, "with advance the positions are the lengths: no start positions")
    assert call(cos=P, sin=None, rope_len=8) == (-1, "rotary tables cos/sin [L, D/2] required")
    assert call(cos=P, sin=P, rope_len=0) == (-1, "rotary tables cos/sin [L, D/2] required")
    assert call(D=96) == (-1, "Supported head_dim: 64 or 128")
    assert call(NB=3) == (-1, "B mismatch")
    assert call(page_size=0) == (-1, "page_size mismatch")


def test_c_abi_rejects_bad_arguments_without_a_device():
    lib = _lib.load()
    P = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc, msg = _status_and_message(lib.fa_flash_attn_fwd(
        P, P, P, P, 0, 1, 8, 8, 16, 16, 96, 1, 0, 0, None, None, None))
    assert rc == -1 and msg == "Supported head_dim: 64 or 128"
    rc, msg = _status_and_message(lib.fa_flash_attn_fwd(
        P, P, P, P, 0, 1, 6, 4, 16, 16, 64, 1, 0, 0, None, None, None))
    assert rc == -1 and msg == "H mismatch"
    rc, msg = _status_and_message(lib.fa_flash_attn_fwd(
        P, P, P, P, 7, 1, 8, 8, 16, 16, 64, 1, 0, 0, None, None, None))
    assert rc == -1 and msg == "fp16 or fp32 required"
    # paged: pool batch must equal B without a block table; page_size positive
    rc, msg = _status_and_message(lib.fa_flash_attn_paged_fwd(
        P, P, P, P, 16, P, P, 2, 8, 1, 128, 3, 8, 4, 0, 0, 0, None, None, None, None, 0, 0, None,
        0, None))
    assert rc == -1 and msg == "B mismatch"
    rc, msg = _status_and_message(lib.fa_flash_attn_paged_fwd(
        P, P, P, P, 0, P, P, 2, 8, 1, 128, 2, 8, 4, 0, 0, 0, None, None, None, None, 0, 0, None,
        0, None))
    assert rc == -1 and msg == "page_size mismatch"
    # decode path without its workspace
    rc, msg = _status_and_message(lib.fa_flash_attn_paged_fwd(
        P, P, P, P, 16, P, P, 2, 8, 1, 128, 2, 8, 4, 0, 0, 0, None, None, None, None, 0, 0, None,
        0, None))
    assert rc == -3 and msg.startswith("workspace of")
    rc, msg = _status_and_message(lib.fa_paged_kv_append(
        P, P, P, P, 2, 4, 3, 12, 2, 4, 16, 0, None, None, 0, None))
    assert rc == -1 and msg == "head_dim must be a multiple of 8"
    # rotary variants: tables required; the fused append needs D % 16 == 0
    rc, msg = _status_and_message(lib.fa_flash_attn_paged_rope_fwd(
        P, P, P, P, 16, P, P, 2, 8, 1, 128, 2, 8, 4, 0, 0, 0, None, None, None, None, 0, 0,
        None, 0, None, None, 0, None))
    assert rc == -1 and msg == "rotary tables cos/sin [L, D/2] required"
    rc, msg = _status_and_message(lib.fa_paged_kv_append_rope(
        P, P, P, P, 2, 4, 3, 128, 2, 4, 16, 0, None, None, 0, None, None, 0, None))
    assert rc == -1 and msg == "rotary tables cos/sin [L, D/2] required"
    rc, msg = _status_and_message(lib.fa_paged_kv_append_rope(
        P, P, P, P, 2, 4, 3, 24, 2, 4, 16, 0, None, None, 0, P, P, 64, None))
    assert rc == -1 and msg == "rotary append needs head_dim a multiple of 16"
    # per-token scatter: positions required when there is work; rope tables in pairs
    sc = lib.fa_paged_kv_scatter
    rc, msg = _status_and_message(sc(P, P, P, P, 2, 4, 3, 128, 2, 4, 16, None, None, 0,
                                     None, None, 0, None))
    assert rc == -1 and msg == "positions [B, T] required"
    rc, msg = _status_and_message(sc(P, P, P, P, 2, 4, 3, 128, 2, 4, 16, P, None, 0,
                                     P, None, 64, None))
    assert rc == -1 and msg == "rotary tables cos/sin [L, D/2] required"
    rc, msg = _status_and_message(sc(P, P, P, P, 2, 4, 3, 128, 3, 4, 16, P, None, 0,
                                     None, None, 0, None))
    assert rc == -1 and msg == "B mismatch"
    assert sc(P, P, P, P, 2, 4, 0, 128, 2, 4, 16, None, None, 0, None, None, 0, None) == 0
    # token-major decode (the INT8 engine's cache): shapes, scale, workspace
    tm = lib.fa_decode_token_major
    rc, msg = _status_and_message(tm(P, P, P, P, 5, 40, 8, 96, 0.1, None, 0, P, 1 << 20, None))
    assert rc == -1 and msg == "Supported head_dim: 64 or 128"
    rc, msg = _status_and_message(tm(P, P, P, P, 5, 0, 8, 128, 0.1, None, 0, P, 1 << 20, None))
    assert rc == -1 and msg == "H and KVH must be positive"
    rc, msg = _status_and_message(tm(P, P, P, P, -1, 40, 8, 128, 0.1, None, 0, P, 1 << 20, None))
    assert rc == -1 and msg == "position t out of range"
    rc, msg = _status_and_message(tm(P, P, P, P, 5, 40, 8, 128, float("inf"), None, 0, P, 1 << 20,
                                     None))
    assert rc == -1 and msg == "scale must be finite"
    rc, msg = _status_and_message(tm(P, P, None, P, 5, 40, 8, 128, 0.1, None, 0, P, 1 << 20, None))
    assert rc == -1 and msg == "null tensor pointer"
    rc, msg = _status_and_message(tm(P, P, P, P, 5, 40, 8, 128, 0.1, None, 0, P, 16, None))
    assert rc == -3 and msg.startswith("workspace of")
    # empty work returns OK without any launch
    assert lib.fa_flash_attn_fwd(P, P, P, P, 0, 0, 8, 8, 16, 16, 64, 1, 0, 0, None, None, None) == 0
    assert lib.fa_paged_kv_append(P, P, P, P, 2, 4, 0, 128, 2, 4, 16, 0, None, None, 0, None) == 0


def test_workspace_sizing_depends_on_sizes_only():
    lib = _lib.load()
    # decode (M = 1): partial slots (B*Hk + workgroups) x (heads_per_kv*M rows)
    # x (D + 2) floats (two 256-byte aligned parts) + the (B + 1) unit prefix
    # and the B positions of the fused append;
    # 1024 workgroups unless a batch has fewer than 8 groups of 16 keys per
    # workgroup. A slot holds one KV head's query rows: cfg4's 64/8 heads need
    # 8 rows per slot (6.3 MB), against 64 with no bound (50 MB).
    align = lambda x: -(-x // 256) * 256  # noqa: E731
    slots = 64 * 8 + 1024
    for hpk, rows in ((8, 8), (0, 64), (-3, 64), (100, 64), (5, 5)):
        ws = lib.fa_paged_workspace_bytes(64, 64, 1, 128, 8, 1025, 16, hpk)
        assert ws == align(slots * rows * 128 * 4) + align(slots * rows * 2 * 4) + 129 * 4, hpk
    assert lib.fa_paged_workspace_bytes(64, 64, 1, 128, 8, 1025, 16, 8) < 7_000_000
    # M = 4 query rows per sequence and 5 heads per KV head: 20 rows per slot
    ws = lib.fa_paged_workspace_bytes(64, 40, 4, 128, 8, 1025, 16, 5)
    assert ws == align(slots * 20 * 128 * 4) + align(slots * 20 * 2 * 4) + 129 * 4
    small = lib.fa_paged_workspace_bytes(1, 8, 1, 64, 8, 2, 16, 1)  # 16 units -> 2 workgroups
    assert small == align((8 + 2) * 1 * 64 * 4) + align((8 + 2) * 1 * 2 * 4) + 3 * 4
    # prefill-shaped calls need no workspace
    assert lib.fa_paged_workspace_bytes(4, 40, 2048, 128, 8, 128, 16, 5) == 0
    assert lib.fa_paged_workspace_bytes(1, 8, 1, 96, 8, 4, 16, 1) == 0
    # More than 32 query rows per KV head (M * ceil(Hq/Hk)) with a
    # heads_per_kv bound: the packed prefill layout (no workspace) once the
    # batch gives 256 tiles of 128 rows (512 while one 64-row decode pass
    # would do), below that the decode kernels in passes of up to 64 rows (at
    # most 256 rows); without a bound, one decode pass or the per-head
    # prefill layout.
    for B, M, hpk, decode in ((64, 16, 8, False), (32, 16, 8, False), (16, 16, 8, True),
                              (2, 32, 8, True), (2, 33, 8, False), (64, 8, 8, False),
                              (32, 8, 8, True), (64, 4, 8, True), (2, 16, 0, False),
                              (64, 8, 0, True)):
        ws = lib.fa_paged_workspace_bytes(B, 64, M, 128, 8, 1025, 16, hpk)
        assert (ws > 0) == decode, (B, M, hpk)
    # token-major decode: one sequence of t_max + 1 keys, 256 groups x 8 KV
    # heads = 2048 units -> 256 workgroups. With an even KV-head count and at
    # most 8 heads per KV head, each segment serves a pair of KV heads: 4
    # segments + 256 slots of 2 x 5 rows. Without a bound (H = 40 rows per KV
    # head, too many to pair) 8 segments + 256 slots of 40 rows.
    t_max = 4095
    ws = lib.fa_decode_token_major_workspace_bytes(40, 8, 128, t_max, 5)
    assert ws == align((4 + 256) * 10 * 128 * 4) + align((4 + 256) * 10 * 2 * 4) + 3 * 4
    ws0 = lib.fa_decode_token_major_workspace_bytes(40, 8, 128, t_max, 0)   # no bound: H rows
    slots = 8 + 256
    assert ws0 == align(slots * 40 * 128 * 4) + align(slots * 40 * 2 * 4) + 3 * 4
    # odd KV-head count (3: 768 units, 96 workgroups) or 9 heads per KV head: no pairs
    assert lib.fa_decode_token_major_workspace_bytes(12, 3, 64, t_max, 4) == (
        align((3 + 96) * 4 * 64 * 4) + align((3 + 96) * 4 * 2 * 4) + 3 * 4)
    assert lib.fa_decode_token_major_workspace_bytes(72, 8, 128, t_max, 9) == (
        align(slots * 9 * 128 * 4) + align(slots * 9 * 2 * 4) + 3 * 4)
    assert lib.fa_decode_token_major_workspace_bytes(40, 8, 128, 100, 5) < ws
    assert lib.fa_decode_token_major_workspace_bytes(40, 8, 96, t_max, 5) == 0
    # a batch beyond 2048 sequences: decode launches of at most 2048, one
    # workspace sized for one of them
    big = lib.fa_paged_workspace_bytes(5000, 8, 1, 64, 2, 64, 16, 4)
    assert big == lib.fa_paged_workspace_bytes(2048, 8, 1, 64, 2, 64, 16, 4) > 0


def test_contiguous_workspace_sizing():
    """fa_flash_attn_workspace_bytes: fp16 calls with at most 32 query rows
    per K/V head take the decode kernels (workspace as for the paged entry
    with heads_per_kv = Hq/Hk and the key count N as the capacity); fp32,
    more rows, N == 0 or an unsupported head_dim need none."""
    lib = _lib.load()
    F16, F32 = _lib.FA_DTYPE_F16, _lib.FA_DTYPE_F32
    ws = lib.fa_flash_attn_workspace_bytes(F16, 4, 40, 8, 1, 4096, 128)
    assert ws == lib.fa_paged_workspace_bytes(4, 40, 1, 128, 8, 256, 16, 5) > 0
    assert lib.fa_flash_attn_workspace_bytes(F16, 2, 8, 8, 4, 300, 64) > 0    # MHA, M = 4
    assert lib.fa_flash_attn_workspace_bytes(F16, 2, 8, 8, 33, 300, 64) == 0  # 33 rows
    assert lib.fa_flash_attn_workspace_bytes(F16, 1, 64, 8, 8, 300, 128) == 0  # 64 rows
    assert lib.fa_flash_attn_workspace_bytes(F32, 4, 40, 8, 1, 4096, 128) == 0
    assert lib.fa_flash_attn_workspace_bytes(F16, 4, 40, 8, 1, 0, 128) == 0
    assert lib.fa_flash_attn_workspace_bytes(F16, 4, 40, 8, 1, 64, 96) == 0
    P = ctypes.c_void_p(16)  # never dereferenced: the workspace check comes first
    rc, msg = _status_and_message(lib.fa_flash_attn_fwd_ws(
        P, P, P, P, F16, 4, 40, 8, 1, 4096, 128, 0, 0, 0, None, None, None, 0, None))
    assert rc == -3 and msg.startswith("workspace of"), msg


def test_heads_per_kv_of_a_head_map():
    """The bound the Python operators pass: the most q heads one KV head
    serves, read once per head-map tensor and refreshed when it changes."""
    from hrm_flashrenderer_amd.ops import heads_per_kv
    hm = (torch.arange(64) // 8).to(torch.int32)
    assert heads_per_kv(hm, 8) == 8
    hm2 = torch.tensor([2, 0, 2, 1, 2, 0], dtype=torch.int32)
    assert heads_per_kv(hm2, 3) == 3
    hm2[0] = 1                              # in-place change: read again
    assert heads_per_kv(hm2, 3) == 2
    assert heads_per_kv(torch.tensor([5, -1, 7], dtype=torch.int32), 3) == 1  # invalid entries


def test_heads_per_kv_of_an_inference_tensor():
    """A head map made under torch.inference_mode() has no version counter:
    the bound is read from it on every call (an in-place edit inside
    inference mode is seen), and no RuntimeError escapes."""
    from hrm_flashrenderer_amd.ops import heads_per_kv
    with torch.inference_mode():
        hm = torch.tensor([2, 0, 2, 1, 2, 0], dtype=torch.int32)
        assert hm.is_inference()
        assert heads_per_kv(hm, 3) == 3
        hm[0] = 1
        assert heads_per_kv(hm, 3) == 2
    assert heads_per_kv(hm, 3) == 2  # outside inference mode too


def test_stated_heads_per_kv_skips_the_map():
    """heads_per_kv= on the operators: a stated bound is used as given (no
    read-back) and must be at least 1."""
    from hrm_flashrenderer_amd.ops import _resolve_heads_per_kv
    hm = torch.tensor([0, 0, 0, 1], dtype=torch.int32)
    assert _resolve_heads_per_kv(None, hm, 2) == 3
    assert _resolve_heads_per_kv(5, hm, 2) == 5
    with pytest.raises(RuntimeError, match="heads_per_kv must be >= 1"):
        _resolve_heads_per_kv(0, hm, 2)
    for fn in (ops.flash_attn_paged, ops.flash_attn_paged_append):
        p = inspect.signature(fn).parameters["heads_per_kv"]
        assert p.kind is inspect.Parameter.KEYWORD_ONLY and p.default is None


def test_no_alloc_entry_rejects_shapes_beyond_its_scratch():
    """fa_flash_attn_paged_fwd_noalloc refuses a decode call whose partial
    results exceed its 32 MiB static scratch, before anything touches a device
    (the pointers are never dereferenced)."""
    lib = _lib.load()
    P = ctypes.c_void_p(16)
    need = lib.fa_paged_workspace_bytes(2048, 64, 1, 128, 8, 2049, 16, 8)
    assert need > 32 << 20
    rc = lib.fa_flash_attn_paged_fwd_noalloc(P, P, P, P, 16, P, P, 2048, 64, 1, 128, 1, 8, 40000,
                                              0, 0, 0, None, None, None, P, 2049, 8, None)
    msg = lib.fa_last_error().decode()
    assert rc == -3 and "allocation-free entry holds 33554432" in msg, msg


def test_signatures_match_reference():
    # flashattention_custom/ops.py:81, 88-90, 97
    def params(fn):
        return [(p.name, p.default) for p in inspect.signature(fn).parameters.values()
                if p.kind is not inspect.Parameter.KEYWORD_ONLY]
    E = inspect.Parameter.empty
    assert params(ops.flash_attn) == [("q", E), ("k", E), ("v", E), ("causal", True),
                                      ("q_offset", 0), ("k_offset", 0)]
    assert params(ops.flash_attn_paged) == [
        ("q", E), ("k_pages", E), ("v_pages", E), ("seqlen", E), ("page_size", E),
        ("head_map", E), ("causal", True), ("q_offset", 0), ("k_offset", 0)]
    assert params(ops.paged_kv_append) == [("k_pages", E), ("v_pages", E), ("k_new", E),
                                           ("v_new", E), ("start_pos", E), ("page_size", E)]
    import flashattention_custom
    import flashattention_custom.ops as alias
    assert alias.flash_attn_paged is ops.flash_attn_paged
    assert flashattention_custom.__all__ == ["flash_attn", "flash_attn_paged", "paged_kv_append"]


def test_cpu_tensors_are_rejected_not_computed():
    q = torch.zeros(1, 8, 4, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="q/k/v must be CUDA"):
        ops.flash_attn(q, q, q)
    kp = torch.zeros(1, 8, 1, 16, 64, dtype=torch.float16)
    sl = torch.zeros(1, dtype=torch.int32)
    hm = torch.arange(8, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="CUDA required"):
        ops.flash_attn_paged(q, kp, kp, sl, 16, hm)
    with pytest.raises(RuntimeError, match="CUDA required"):
        ops.paged_kv_append(kp, kp, q[:, :, :1], q[:, :, :1], 0, 16)


def _f16(*s):
    return torch.zeros(*s, dtype=torch.float16)


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(k=a["k"].float()), "fp16 required"),
    (lambda a: a.update(q=_f16(1, 8, 64, 4).transpose(2, 3)), "contiguous required"),
    (lambda a: a.update(q=_f16(8, 4, 64)), "q/k/v must be 4D"),
    (lambda a: a.update(k=_f16(2, 8, 6, 64), v=_f16(2, 8, 6, 64)), "B mismatch"),
    (lambda a: a.update(k=_f16(1, 3, 6, 64), v=_f16(1, 3, 6, 64)), "H mismatch"),
    (lambda a: a.update(v=_f16(1, 8, 7, 64)), "N mismatch"),
    (lambda a: a.update(q=_f16(1, 8, 4, 32)), "D mismatch"),
    (lambda a: a.update(q=_f16(1, 8, 4, 96), k=_f16(1, 8, 6, 96), v=_f16(1, 8, 6, 96)),
     "Supported head_dim: 64 or 128"),
])
def test_flash_attn_validation_messages(mutate, msg):
    a = dict(q=_f16(1, 8, 4, 64), k=_f16(1, 8, 6, 64), v=_f16(1, 8, 6, 64))
    ops.validate_flash_attn(**a, require_device=False)
    mutate(a)
    with pytest.raises(RuntimeError, match=msg):
        ops.validate_flash_attn(**a, require_device=False)


def _paged_args():
    return dict(q=_f16(2, 8, 1, 128), k_pages=_f16(2, 2, 4, 16, 128),
                v_pages=_f16(2, 2, 4, 16, 128), seqlen=torch.zeros(2, dtype=torch.int32),
                page_size=16, head_map=(torch.arange(8) // 4).to(torch.int32))


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(v_pages=a["v_pages"].float()), "fp16 required"),
    (lambda a: a.update(seqlen=a["seqlen"].long()), "seqlen int32 required"),
    (lambda a: a.update(head_map=a["head_map"].long()), "head_map int32 required"),
    (lambda a: a.update(q=_f16(2, 8, 2, 128)[:, :, :1]), "contiguous required"),
    (lambda a: a.update(q=_f16(2, 8, 128)), r"q \[B,Hq,M,D\]"),
    (lambda a: a.update(k_pages=_f16(2, 2, 64, 128)), r"k_pages/v_pages \[B,Hk,P,PS,D\]"),
    (lambda a: a.update(v_pages=_f16(2, 2, 5, 16, 128)), "k_pages/v_pages mismatch"),
    (lambda a: a.update(q=_f16(3, 8, 1, 128)), "B mismatch"),
    (lambda a: a.update(head_map=torch.zeros(7, dtype=torch.int32)), "Hq mismatch"),
    (lambda a: a.update(page_size=32), "page_size mismatch"),
    (lambda a: a.update(q=_f16(2, 8, 1, 64)), "D mismatch"),
    (lambda a: a.update(seqlen=torch.zeros(1, dtype=torch.int32)), r"seqlen \[B\] required"),
    (lambda a: a.update(block_table=torch.zeros(3, 4, dtype=torch.int32)),
     r"block_table \[B, max_blocks\] required"),
    (lambda a: a.update(block_table=torch.zeros(2, 4, dtype=torch.int64)),
     "block_table int32 required"),
])
def test_flash_attn_paged_validation_messages(mutate, msg):
    a = _paged_args()
    ops.validate_flash_attn_paged(**a, require_device=False)
    mutate(a)
    with pytest.raises(RuntimeError, match=msg):
        ops.validate_flash_attn_paged(**a, require_device=False)


def test_block_table_allows_a_shared_pool():
    a = _paged_args()
    a.update(k_pages=_f16(1, 2, 9, 16, 128), v_pages=_f16(1, 2, 9, 16, 128),
             block_table=torch.zeros(2, 5, dtype=torch.int32))
    assert ops.validate_flash_attn_paged(**a, require_device=False) == 5


def _append_args():
    return dict(k_pages=_f16(2, 4, 8, 128, 128), v_pages=_f16(2, 4, 8, 128, 128),
                k_new=_f16(2, 4, 96, 128), v_new=_f16(2, 4, 96, 128), start_pos=145,
                page_size=128)


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(k_new=a["k_new"].float()), "fp16 required"),
    (lambda a: a.update(k_pages=_f16(2, 4, 8, 128, 128).transpose(0, 1)), "contiguous required"),
    (lambda a: a.update(k_new=_f16(2, 4, 96 * 128)), "shape mismatch"),
    (lambda a: a.update(v_pages=_f16(2, 4, 9, 128, 128)), "k_pages/v_pages mismatch"),
    (lambda a: a.update(v_new=_f16(2, 4, 95, 128)), "k_new/v_new mismatch"),
    (lambda a: a.update(k_new=_f16(3, 4, 96, 128), v_new=_f16(3, 4, 96, 128)), "B mismatch"),
    (lambda a: a.update(k_new=_f16(2, 2, 96, 128), v_new=_f16(2, 2, 96, 128)), "Hk mismatch"),
    (lambda a: a.update(page_size=64), "page_size mismatch"),
    (lambda a: a.update(k_new=_f16(2, 4, 96, 64), v_new=_f16(2, 4, 96, 64)), "D mismatch"),
    (lambda a: a.update(start_pos=8 * 128 - 95), "exceeds the page capacity"),
    (lambda a: a.update(start_pos=-1), "exceeds the page capacity"),
    (lambda a: a.update(start_pos=torch.zeros(3, dtype=torch.int32)), r"start_pos \[B\] required"),
])
def test_paged_kv_append_validation_messages(mutate, msg):
    a = _append_args()
    assert ops.validate_paged_kv_append(**a, require_device=False) == (145, None)
    mutate(a)
    with pytest.raises(RuntimeError, match=msg):
        ops.validate_paged_kv_append(**a, require_device=False)


def test_custom_ops_have_shape_functions():
    q = torch.empty(2, 8, 3, 128, dtype=torch.float16, device="meta")
    kp = torch.empty(2, 2, 4, 16, 128, dtype=torch.float16, device="meta")
    sl = torch.empty(2, dtype=torch.int32, device="meta")
    hm = torch.empty(8, dtype=torch.int32, device="meta")
    o = torch.ops.hrm_fa.flash_attn_paged(q, kp, kp, sl, 16, hm, True, 0, 0, None, None, None,
                                          None, None)
    assert o.shape == q.shape and o.dtype == q.dtype
    cs = torch.empty(64, 64, dtype=torch.float16, device="meta")
    o = torch.ops.hrm_fa.flash_attn_paged(q, kp, kp, sl, 16, hm, True, 0, 0, None, None, None,
                                          cs, cs)
    assert o.shape == q.shape
    o2 = torch.ops.hrm_fa.flash_attn(q, q, q, True, 0, 0, None, None)
    assert o2.shape == q.shape
    kn = torch.empty(2, 2, 1, 128, dtype=torch.float16, device="meta")
    assert torch.ops.hrm_fa.paged_kv_append(kp, kp, kn, kn, 0, None, 16, None, None, None) is None
    assert torch.ops.hrm_fa.paged_kv_append(kp, kp, kn, kn, 0, None, 16, None, cs, cs) is None


def test_product_path_does_not_import_the_oracle():
    pkg = os.path.join(REPO, "hrm_flashrenderer_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(root, f)).read()
                assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", src, re.M), f


@pytest.mark.parametrize("rope,msg", [
    ((_f16(8, 64),), "rope must be"),
    ((_f16(8, 32), _f16(8, 32)), r"cos/sin \[L, D/2\]"),
    ((_f16(8, 64), _f16(9, 64)), r"cos/sin \[L, D/2\]"),
    ((torch.zeros(8, 64), torch.zeros(8, 64)), "fp16 required"),
    ((_f16(64, 8).t(), _f16(64, 8).t()), "contiguous required"),
])
def test_rope_table_validation(rope, msg):
    with pytest.raises(RuntimeError, match=msg):
        ops._check_rope(rope, 128, torch.device("cpu"), require_device=False)
    assert ops._check_rope(None, 128, torch.device("cpu"), require_device=False) == (None, None)


def _integration_shim_namespace(real: bool = False):
    """Executes the `_ext` binding that the repository's integration guide
    prints (its `flashattention_custom/_ext.py` block) against the built
    library. Unless `real`, it then swaps the shim's library handle for one
    that fails any compute call, so a test sees whether validation happens
    first."""
    guide = "INTEGRATION.md"
    text = open(os.path.join(REPO, guide)).read()
    start = text.index("```python\n# flashattention_custom/_ext.py — binds")
    code = text[start + len("```python\n"):text.index("```", start + 10)]
    old = os.environ.get("FA_MI355X_LIB")
    os.environ["FA_MI355X_LIB"] = _lib.LIB_PATH
    try:
        ns = {}
        exec(compile(code, guide + ":_ext.py", "exec"), ns)
    finally:
        if old is None:
            os.environ.pop("FA_MI355X_LIB", None)
        else:
            os.environ["FA_MI355X_LIB"] = old

    class NoCompute:
        def __getattr__(self, name):
            raise AssertionError(f"C entry {name} reached before validation")
    if not real:
        ns["_LIB"] = NoCompute()
    return ns


def test_integration_shim_validates_before_the_c_call():
    ns = _integration_shim_namespace()
    q = torch.zeros(1, 8, 16, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="q/k/v must be CUDA"):
        ns["flash_attn_fwd"](q, q, q)
    kp = torch.zeros(1, 8, 2, 16, 64, dtype=torch.float16)
    sl = torch.zeros(1, dtype=torch.int32)
    hm = torch.zeros(8, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="CUDA required"):
        ns["flash_attn_paged_fwd"](q, kp, kp, sl, 16, hm)
    k1 = torch.zeros(1, 8, 1, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="CUDA required"):
        ns["paged_kv_append"](kp, kp, k1, k1, 0, 16)
