"""C-ABI checks that need no GPU: the library loads, exports every function
declared in include/parrot_hip.h, and rejects bad arguments with the
documented negative status before any HIP call is made."""
import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "parrot_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(parrot_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from parrot import _abi
    if not _abi.LIBRARY.exists():
        pytest.fail("libparrot_hip.so is not built; run __graft_entry__.build()")
    return _abi.load()


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    assert "parrot_route_bf16" in names and "parrot_grouped_experts_bf16" in names
    from parrot import _abi
    assert names == sorted(_abi.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    from parrot import _abi
    for name in _declared_functions():
        assert hasattr(lib, name), name
        assert name in _abi.SIGNATURES, f"{name} missing from the ctypes binding"


def test_version_and_status_strings(lib):
    from parrot import _abi
    header = (ROOT / "include" / "parrot_hip.h").read_text()
    assert f"#define PARROT_ABI_VERSION {_abi.ABI_VERSION}" in header
    assert lib.parrot_abi_version() == _abi.ABI_VERSION
    assert lib.parrot_status_string(0) == b"ok"
    for code in (-1, -2, -3, -4, -5, -6):
        assert lib.parrot_status_string(code) != b"unknown status"


def test_capacity_matches_oracle(lib):
    from oracle import routing
    for tokens in (0, 1, 8, 64, 255, 256, 512, 4096, 10007):
        for experts in (2, 8, 16, 32):
            assert lib.parrot_capacity(tokens, experts) == routing.capacity(tokens, experts)


def test_workspace_sizes(lib):
    # one int32 histogram row of E counts per 16-token route block ...
    assert lib.parrot_route_workspace_bytes(512, 16) >= 32 * 16 * 4
    assert lib.parrot_route_workspace_bytes(4096, 16) >= 256 * 16 * 4
    # ... plus one row per 256 route blocks once there is more than one chunk
    assert lib.parrot_route_workspace_bytes(65536, 16) >= (4096 + 16) * 16 * 4
    assert lib.parrot_route_workspace_bytes(4097, 32) >= (257 + 2) * 32 * 4
    small = lib.parrot_experts_workspace_bytes(8, 768, 512, 256)
    big = lib.parrot_experts_workspace_bytes(512, 768, 512, 256)
    assert big > small > 0
    # hidden rows [3T, max(H, Hs)] and the bf16 expert outputs [3T, dim]
    assert big >= 3 * 512 * 512 * 2 + 3 * 512 * 768 * 2


def test_decode_heads_predicate(lib):
    """The deferred decode step's shape predicate (hip_moe.
    decode_attention_heads_supported, the C ABI's
    parrot_decode_attention_heads_check): the default model's local layers
    defer at one to four rows; more than 16 query heads (one pending lane
    each), a window whose scores overflow the heads kernel's LDS, or more
    rows take the undeferred decode."""
    from parrot import hip_moe
    default = dict(dim=768, heads=8, kv_heads=2, head_dim=96, max_positions=4096, window=2048)
    for tokens in (1, 2, 4):
        assert hip_moe.decode_attention_heads_supported(tokens, **default)
    assert not hip_moe.decode_attention_heads_supported(5, **default)
    assert not hip_moe.decode_attention_heads_supported(0, **default)
    assert hip_moe.decode_attention_heads_supported(1, **{**default, "heads": 16})
    assert not hip_moe.decode_attention_heads_supported(
        1, **{**default, "heads": 32, "kv_heads": 4, "head_dim": 32})
    # 16000 fp32 scores alone fill the 64 KB of LDS
    assert not hip_moe.decode_attention_heads_supported(
        1, **{**default, "max_positions": 16384, "window": 16000})
    assert hip_moe.decode_attention_heads_supported(
        1, **{**default, "max_positions": 16384, "window": 8192})
    assert not hip_moe.decode_attention_heads_supported(1, **{**default, "dim": 776})
    assert not hip_moe.decode_attention_heads_supported(1, **{**default, "dim": 2048})
    assert lib.parrot_decode_attention_heads_check(1, 32, 4, 32, 4096, 2048, 768) == -3
    assert lib.parrot_decode_attention_heads_check(1, 8, 3, 96, 4096, 2048, 768) == -3
    assert lib.parrot_decode_attention_heads_check(1, 8, 2, 96, 4096, 0, 768) == -2
    assert lib.parrot_decode_attention_heads_check(1, 8, 2, 96, 4096, 2048, 768) == 0


def test_argument_validation_without_gpu(lib):
    """Rejected before launch: no device is touched."""
    from parrot import _abi
    for name, (_, argtypes) in _abi.SIGNATURES.items():
        assert len(argtypes) == len(getattr(lib, name).argtypes)
    fake = 0x10000  # 16-byte aligned, never dereferenced on these paths
    null = None
    assert lib.parrot_rms_norm_bf16(null, fake, fake, 4, 64, 1e-6, null) == -1
    assert lib.parrot_rms_norm_bf16(fake, fake, fake, 4, 66, 1e-6, null) == -2
    assert lib.parrot_rms_norm_bf16(fake, fake, fake, 4, 8192, 1e-6, null) == -3
    assert lib.parrot_rms_norm_bf16(fake + 2, fake, fake, 4, 64, 1e-6, null) == -5
    srcs = (ctypes.c_void_p * 9)(*([fake] * 9))
    assert lib.parrot_depth_mix_bf16(ctypes.cast(srcs, ctypes.c_void_p), 10, fake, fake, 1e-6,
                                     fake, 1e-6, 4, 64, fake, null, null) == -3
    assert lib.parrot_depth_mix_bf16(ctypes.cast(srcs, ctypes.c_void_p), 2, fake, fake, 1e-6,
                                     null, 1e-6, 4, 64, null, null, null) == -1
    # the forward's first launch: shapes, pointers and alignment
    assert lib.parrot_embed_depth_mix_bf16(fake, 4, fake, 100, 66, fake, fake, 1e-6, fake,
                                           1e-6, fake, fake, null, 0, null) == -2
    assert lib.parrot_embed_depth_mix_bf16(fake, 4, fake, 100, 4096, fake, fake, 1e-6, fake,
                                           1e-6, fake, fake, null, 0, null) == -3
    assert lib.parrot_embed_depth_mix_bf16(fake, 4, null, 100, 64, fake, fake, 1e-6, fake,
                                           1e-6, fake, fake, null, 0, null) == -1
    assert lib.parrot_embed_depth_mix_bf16(fake, 4, fake, 100, 64, fake, fake, 1e-6, fake,
                                           1e-6, fake, fake, null, 8, null) == -1
    assert lib.parrot_embed_depth_mix_bf16(fake, 4, fake, 0, 64, fake, fake, 1e-6, fake,
                                           1e-6, fake, fake, null, 0, null) == -2
    assert lib.parrot_embed_depth_mix_bf16(fake, 4, fake + 2, 100, 64, fake, fake, 1e-6, fake,
                                           1e-6, fake, fake, null, 0, null) == -5
    # attention with the output projection deferred per head: widths, shapes
    ost = (ctypes.c_int64 * 3)(8 * 512 * 96, 512 * 96, 96)
    attn_out = lambda **kw: lib.parrot_causal_attention_frag_out_bf16(*[kw.get(k, v) for k, v in (
        ("q", fake), ("st", ctypes.cast(ost, ctypes.c_void_p)), ("kf", fake), ("vf", fake),
        ("b", 1), ("t", 512), ("h", 8), ("hk", 2), ("d", 96), ("win", 2048), ("sc", 0.1),
        ("w", fake), ("dim", 768), ("out", fake), ("stream", null))])
    assert attn_out(w=null) == -1 and attn_out(out=null) == -1
    assert attn_out(dim=0) == -2 and attn_out(win=0) == -2
    assert attn_out(dim=640) == -3 and attn_out(d=80) == -3 and attn_out(h=6, hk=4) == -3
    assert attn_out(w=fake + 8) == -5 and attn_out(out=fake + 4) == -5
    # the MoE input mix with a pending attention output: 8 heads, 2+ sources
    srcs2 = (ctypes.c_void_p * 9)(*([fake] * 9))
    pend = lambda **kw: lib.parrot_depth_mix_route_pending_bf16(*[kw.get(k, v) for k, v in (
        ("src", ctypes.cast(srcs2, ctypes.c_void_p)), ("n", 3), ("q", fake), ("sw", fake),
        ("se", 1e-6), ("nw", fake), ("ne", 1e-6), ("tokens", 4), ("dim", 768), ("out", fake),
        ("rw", fake), ("bias", null), ("e", 16), ("wts", fake), ("idx", fake), ("c", fake),
        ("heads", 8), ("base", null), ("res", fake), ("stream", null))])
    assert pend(c=null) == -1 and pend(res=null) == -1 and pend(out=null) == -1
    assert pend(heads=4) == -3 and pend(n=1) == -3 and pend(e=33) == -3 and pend(dim=776) == -3
    assert pend(c=fake + 8) == -5 and pend(res=fake + 2) == -5
    ws = lib.parrot_route_workspace_bytes(64, 8)
    args = [fake] * 9  # out_logits .. out_overflow
    # experts outside 2..32
    assert lib.parrot_route_bf16(fake, fake, null, 64, 64, 33, 32, *args, fake, ws, null) == -3
    # dim not a multiple of 32
    assert lib.parrot_route_bf16(fake, fake, null, 64, 48, 8, 32, *args, fake, ws, null) == -3
    # workspace too small
    assert lib.parrot_route_bf16(fake, fake, null, 64, 64, 8, 32, *args, fake, 0, null) == -4
    # grouped experts: widths must be multiples of 64
    assert lib.parrot_grouped_experts_bf16(
        fake, 64, 96, 8, 128, 64, 32, *([fake] * 9), null, fake, fake, 1 << 30, null) == -3
    assert lib.parrot_grouped_experts_bf16(
        fake, 64, 64, 8, 128, 64, 32, *([fake] * 9), null, fake, fake, 16, null) == -4
    # RoPE: start + seq past the table
    assert lib.parrot_rope_qkv_bf16(fake, fake, fake, 1, 4, 126, null, 128, 8, 2, 96, 0, 0,
                                    fake, fake, fake, null) == -2
    # RoPE: transposed values need room for every key and no kv expansion
    assert lib.parrot_rope_qkv_bf16(fake, fake, fake, 1, 40, 0, null, 128, 8, 2, 96, 0, 32,
                                    fake, fake, fake, null) == -2
    assert lib.parrot_rope_qkv_bf16(fake, fake, fake, 1, 4, 0, null, 128, 8, 2, 96, 1, 32,
                                    fake, fake, fake, null) == -2
    # causal attention: unsupported head width, short V^T rows, odd strides
    st = (ctypes.c_int64 * 3)(8 * 512 * 96, 512 * 96, 96)
    vt_ok = (ctypes.c_int64 * 3)(2 * 96 * 512, 96 * 512, 512)
    vt_short = (ctypes.c_int64 * 3)(2 * 96 * 496, 96 * 496, 496)
    odd = (ctypes.c_int64 * 3)(8 * 512 * 96, 512 * 96, 100)

    def attn(q_st=st, vt_st=vt_ok, d=96, seq=512):
        return lib.parrot_causal_attention_bf16(
            fake, fake, fake, ctypes.cast(q_st, ctypes.c_void_p), ctypes.cast(st, ctypes.c_void_p),
            ctypes.cast(vt_st, ctypes.c_void_p), 1, seq, 8, 2, d, 2048, 0.1, fake, null)
    assert attn(d=80) == -3
    assert attn(vt_st=vt_short) == -2
    assert attn(q_st=odd) == -5
    # decode attention: null position, head_dim % 8, heads % kv_heads, LDS budget, alignment
    dec = dict(batch=2, heads=8, kv_heads=2, head_dim=96, max_positions=4096, window=2048)

    def local(position=fake, k_new=fake, **kw):
        a = {**dec, **kw}
        return lib.parrot_decode_attention_bf16(
            fake, k_new, fake, fake, fake, position, a["batch"], a["heads"], a["kv_heads"],
            a["head_dim"], a["max_positions"], a["window"], 0.1, fake, null)
    assert local(position=null) == -1
    assert local(head_dim=100) == -3
    assert local(head_dim=264) == -3
    assert local(heads=6, kv_heads=4) == -3
    assert local(window=0) == -2
    assert local(window=1 << 20, max_positions=1 << 20) == -3
    assert local(k_new=fake + 8) == -5
    assert lib.parrot_decode_attention_latent_f32(fake, fake, fake, null, 2, 8, 128, 4096, 0.1,
                                                  fake, null) == -1
    assert lib.parrot_decode_attention_latent_f32(fake, fake, fake, fake, 2, 8, 128, 1 << 16,
                                                  0.1, fake, null) == -3
    # decode q|k|v: x or sources, tokens <= 16, dim % 128 <= 1024, head_dim even
    qkv = lambda **kw: lib.parrot_decode_qkv_bf16(*[kw.get(k, v) for k, v in (
        ("x", fake), ("srcs", null), ("n", 0), ("q0", null), ("sw", null), ("se", 1e-6),
        ("nw", null), ("ne", 1e-6), ("tokens", 2), ("dim", 768), ("w", fake), ("h", 8),
        ("hk", 2), ("d", 96), ("cos", fake), ("sin", fake), ("maxp", 4096), ("pos", fake),
        ("q", fake), ("k", fake), ("v", fake), ("stream", null))])
    assert qkv(x=null) == -1 and qkv(pos=null) == -1 and qkv(v=null) == -1
    assert qkv(x=null, srcs=ctypes.cast(srcs, ctypes.c_void_p), n=2) == -1  # query missing
    assert qkv(tokens=-1) == -2 and qkv(d=0) == -2 and qkv(maxp=0) == -2
    assert qkv(tokens=17) == -3 and qkv(dim=1152) == -3 and qkv(dim=704) == -3
    assert qkv(d=95) == -3 and qkv(h=3, hk=1, d=6) == -3
    assert qkv(w=fake + 8) == -5
    # ... with the embedding gather: ids, table, row buffer, vocab > 0
    embed = lambda **kw: lib.parrot_decode_qkv_embed_bf16(*[kw.get(k, v) for k, v in (
        ("ids", fake), ("table", fake), ("vocab", 1000), ("rows", fake), ("q0", fake),
        ("sw", fake), ("se", 1e-6), ("nw", fake), ("ne", 1e-6), ("tokens", 2), ("dim", 768),
        ("w", fake), ("h", 8), ("hk", 2), ("d", 96), ("cos", fake), ("sin", fake),
        ("maxp", 4096), ("pos", fake), ("q", fake), ("k", fake), ("v", fake), ("stream", null))])
    assert embed(ids=null) == -1 and embed(rows=null) == -1 and embed(q0=null) == -1
    assert embed(vocab=0) == -2 and embed(tokens=17) == -3 and embed(dim=1152) == -3
    assert embed(table=fake + 8) == -5 and embed(rows=fake + 2) == -5
    # decode MoE with its input's depth mix: sources, n_sources, dim <= 1024
    mix_moe = lambda **kw: lib.parrot_depth_mix_decode_moe_bf16(*[kw.get(k, v) for k, v in (
        ("srcs", ctypes.cast(srcs, ctypes.c_void_p)), ("n", 2), ("q", fake), ("sw", fake),
        ("se", 1e-6), ("nw", fake), ("ne", 1e-6), ("tokens", 2), ("dim", 768), ("e", 16),
        ("h", 512), ("hs", 256), ("rw", fake), ("bias", null), ("gu", fake), ("dn", fake),
        ("sgu", fake), ("sdn", fake), ("add", null), ("out", fake), ("idx", fake),
        ("w", fake), ("ws", fake), ("wsb", 1 << 20), ("stream", null))])
    assert mix_moe(srcs=null) == -1 and mix_moe(q=null) == -1 and mix_moe(nw=null) == -1
    assert mix_moe(n=0) == -3 and mix_moe(n=10) == -3 and mix_moe(dim=1088) == -3
    assert mix_moe(tokens=17) == -3 and mix_moe(wsb=16) == -4
    assert mix_moe(q=fake + 4) == -5
    # MLA decode projections: tokens <= 16, K % 128 <= 2048, rows % 16,
    # staged input <= 64 KB, alignment
    mla_in = lambda **kw: lib.parrot_mla_decode_in_bf16(*[kw.get(k, v) for k, v in (
        ("x", fake), ("srcs", null), ("n", 0), ("q0", null), ("sw", null), ("se", 1e-6),
        ("nw", null), ("ne", 1e-6), ("tokens", 2), ("dim", 768), ("wq", fake), ("nq", 1024),
        ("wkv", fake), ("nl", 128), ("q", fake), ("lat", fake), ("stream", null))])
    assert mla_in(x=null) == -1 and mla_in(lat=null) == -1
    assert mla_in(x=null, srcs=ctypes.cast(srcs, ctypes.c_void_p), n=2) == -1  # query missing
    assert mla_in(x=null, srcs=ctypes.cast(srcs, ctypes.c_void_p), n=2, q0=fake, sw=fake,
                  nw=fake, dim=1152) == -3  # the mix holds dim <= 1024
    assert mla_in(tokens=-1) == -2 and mla_in(nq=0) == -2
    assert mla_in(tokens=17) == -3 and mla_in(dim=704) == -3 and mla_in(dim=2176) == -3
    assert mla_in(nq=1000) == -3 and mla_in(nl=120) == -3
    assert mla_in(wq=fake + 8) == -5
    lin = lambda **kw: lib.parrot_decode_linear_bf16(*[kw.get(k, v) for k, v in (
        ("x", fake), ("tokens", 2), ("k", 768), ("w", fake), ("n", 768), ("add", null),
        ("out", fake), ("stream", null))])
    assert lin(x=null) == -1 and lin(out=null) == -1 and lin(n=0) == -2
    assert lin(tokens=17) == -3 and lin(k=700) == -3 and lin(n=760) == -3
    assert lin(k=2176) == -3  # k <= 2048
    assert lin(w=fake + 8) == -5
    mla_out = lambda **kw: lib.parrot_mla_decode_out_bf16(*[kw.get(k, v) for k, v in (
        ("ctx", fake), ("tokens", 2), ("width", 1024), ("wo", fake), ("dim", 768),
        ("addend", null), ("out", fake), ("stream", null))])
    assert mla_out(ctx=null) == -1 and mla_out(out=null) == -1
    assert mla_out(dim=0) == -2
    assert mla_out(width=1000) == -3 and mla_out(dim=760) == -3
    assert mla_out(tokens=16, width=2048) == -3  # 128 KB of staged context
    assert mla_out(wo=fake + 4) == -5
    # dense projections: k % 64, k <= 2048, n % 16, strides and alignment
    assert lib.parrot_proj_bf16(null, 4, 768, 768, fake, 768, null, 0, fake, 768, null) == -1
    assert lib.parrot_proj_bf16(fake, 4, 96, 96, fake, 768, null, 0, fake, 768, null) == -3
    assert lib.parrot_proj_bf16(fake, 4, 4096, 4096, fake, 768, null, 0, fake, 768, null) == -3
    assert lib.parrot_proj_bf16(fake, 4, 768, 768, fake, 24, null, 0, fake, 24, null) == -3
    assert lib.parrot_proj_bf16(fake, 4, 768, 700, fake, 768, null, 0, fake, 768, null) == -2
    assert lib.parrot_proj_bf16(fake, 4, 768, 768, fake, 768, fake, 700, fake, 768, null) == -2
    assert lib.parrot_proj_bf16(fake, 4, 768, 772, fake, 768, null, 0, fake, 768, null) == -5
    assert lib.parrot_proj_bf16(fake + 8, 4, 768, 768, fake, 768, null, 0, fake, 768, null) == -5
    # transposed: room for every key, 4-key rows, 8-byte aligned output
    assert lib.parrot_proj_transposed_bf16(fake, 2, 40, 128, fake, 768, 32, fake, null) == -2
    assert lib.parrot_proj_transposed_bf16(fake, 2, 40, 128, fake, 768, 42, fake, null) == -5
    assert lib.parrot_proj_transposed_bf16(fake, 2, 40, 128, fake, 768, 64, fake + 2,
                                           null) == -5
    # fused q|k|v + RoPE: the RoPE shape rules, the projection shape rules
    assert lib.parrot_proj_rope_qkv_bf16(fake, 1, 4, 768, fake, fake, fake, 126, null, 128, 8,
                                         2, 96, 0, fake, fake, fake, null) == -2
    assert lib.parrot_proj_rope_qkv_bf16(fake, 1, 40, 768, fake, fake, fake, 0, null, 128, 8,
                                         2, 96, 32, fake, fake, fake, null) == -2
    assert lib.parrot_proj_rope_qkv_bf16(fake, 1, 4, 768, fake, fake, fake, 0, null, 128, 8,
                                         2, 98, 0, fake, fake, fake, null) == -3
    assert lib.parrot_proj_rope_qkv_bf16(fake, 1, 4, 800, fake, fake, fake, 0, null, 128, 8,
                                         2, 96, 0, fake, fake, fake, null) == -3
    assert lib.parrot_proj_rope_qkv_bf16(fake, 1, 4, 768, fake, fake, fake, 0, null, 128, 8,
                                         2, 96, 32, fake, fake, fake + 2, null) == -5
    # fragment-order attention and the projections that write it
    st8 = (ctypes.c_int64 * 3)(8 * 512 * 96, 512 * 96, 96)
    st_odd = (ctypes.c_int64 * 3)(8 * 512 * 96, 512 * 96, 100)

    def attn_frag(q_st=st8, d=96, kf=fake, window=2048):
        return lib.parrot_causal_attention_frag_bf16(
            fake, ctypes.cast(q_st, ctypes.c_void_p), kf, fake, 1, 512, 8, 2, d, window, 0.1,
            fake, null)
    assert attn_frag(kf=null) == -1
    assert attn_frag(d=80) == -3
    assert attn_frag(window=0) == -2
    assert attn_frag(q_st=st_odd) == -5
    assert attn_frag(kf=fake + 8) == -5
    assert lib.parrot_proj_rope_qkv_frag_bf16(fake, 1, 4, 768, fake, fake, fake, 0, null, 128, 8,
                                              2, 96, fake, null, null, null, fake, null) == -1
    assert lib.parrot_proj_rope_qkv_frag_bf16(fake, 1, 4, 768, fake, fake, fake, 126, null, 128,
                                              8, 2, 96, fake, null, null, fake, fake, null) == -2
    assert lib.parrot_proj_rope_qkv_frag_bf16(fake, 1, 4, 768, fake, fake, fake, 0, null, 128, 8,
                                              2, 80, fake, null, null, fake, fake, null) == -3
    assert lib.parrot_proj_frag_bf16(fake, 1, 4, 128, fake, 768, 96, 2, fake, null) == -2
    assert lib.parrot_proj_frag_bf16(fake, 1, 4, 128, fake, 770, 96, 0, fake, null) == -2
    assert lib.parrot_proj_frag_bf16(fake, 1, 4, 128, fake, 640, 80, 0, fake, null) == -3
    assert lib.parrot_proj_frag_bf16(fake, 1, 4, 128, fake, 768, 96, 1, fake + 8, null) == -5
    assert lib.parrot_proj_kv_frag_bf16(fake, 1, 4, 128, 896, fake, 768, 96, fake, null,
                                        null) == -1
    assert lib.parrot_proj_kv_frag_bf16(fake, 1, 4, 128, 100, fake, 768, 96, fake, fake,
                                        null) == -2
    assert lib.parrot_proj_kv_frag_bf16(fake, 1, 4, 128, 900, fake, 768, 96, fake, fake,
                                        null) == -5
    assert lib.parrot_proj_kv_frag_bf16(fake, 1, 4, 128, 896, fake, 768, 80, fake, fake,
                                        null) == -2
    # combine folded into a depth mix: sources, counts, workspace
    ews = lib.parrot_experts_workspace_bytes(64, 64, 128, 64)
    assert lib.parrot_experts_combine_depth_mix_bf16(
        64, 64, 128, 64, null, fake, fake, ews, null, 2, fake, fake, 1e-6, fake, 1e-6, null, fake,
        null) == -1
    assert lib.parrot_experts_combine_depth_mix_bf16(
        64, 64, 128, 64, null, fake, fake, ews, fake, 10, fake, fake, 1e-6, fake, 1e-6, null,
        fake, null) == -3
    assert lib.parrot_experts_combine_depth_mix_bf16(
        64, 64, 128, 64, null, fake, fake, 16, null, 1, fake, fake, 1e-6, fake, 1e-6, null, fake,
        null) == -4
    # depth mix + route: out_norm and router required, experts 2..32, dim % 32
    assert lib.parrot_depth_mix_route_bf16(
        ctypes.cast(srcs, ctypes.c_void_p), 2, fake, fake, 1e-6, fake, 1e-6, 4, 64, null, null,
        fake, null, 8, fake, fake, null) == -1
    assert lib.parrot_depth_mix_route_bf16(
        ctypes.cast(srcs, ctypes.c_void_p), 2, fake, fake, 1e-6, fake, 1e-6, 4, 64, null, fake,
        fake, null, 33, fake, fake, null) == -3
    assert lib.parrot_depth_mix_route_bf16(
        ctypes.cast(srcs, ctypes.c_void_p), 2, fake, fake, 1e-6, fake, 1e-6, 4, 48, null, fake,
        fake, null, 8, fake, fake, null) == -3
    assert lib.parrot_depth_mix_route_bf16(
        ctypes.cast(srcs, ctypes.c_void_p), 2, fake, fake, 1e-6, fake, 1e-6, 4, 64, null, fake,
        fake + 8, null, 8, fake, fake, null) == -5
    # in-kernel grouping: which shapes, and its entry points' checks
    # 1: from the ids; 2: from the route block table only; 0: neither
    assert lib.parrot_experts_group_in_kernel(512, 768, 16, 512, 256) == 1
    assert lib.parrot_experts_group_in_kernel(1024, 768, 32, 512, 256) == 1
    assert lib.parrot_experts_group_in_kernel(1025, 768, 32, 512, 256) == 2  # > 2048 ids
    assert lib.parrot_experts_group_in_kernel(1024, 768, 16, 512, 256) == 2  # 128 rows/expert
    assert lib.parrot_experts_group_in_kernel(4096, 768, 32, 512, 256) == 2  # config 3
    assert lib.parrot_experts_group_in_kernel(4097, 768, 32, 512, 256) == 0  # > 256 blocks
    assert lib.parrot_experts_group_in_kernel(4096, 768, 16, 512, 256) == 0  # wide tiles
    assert lib.parrot_experts_group_in_kernel(512, 1024, 16, 512, 256) == 0  # dim > 768
    assert lib.parrot_experts_group_in_kernel(512, 768, 33, 512, 256) == 0
    # the route block table: T < 32768, 16-byte aligned
    assert lib.parrot_route_top2_blocks_bf16(fake, fake, null, 64, 768, 16, fake, fake, null,
                                             null) == -1
    assert lib.parrot_route_top2_blocks_bf16(fake, fake, null, 32768, 768, 16, fake, fake,
                                             fake, null) == -3
    assert lib.parrot_route_top2_blocks_bf16(fake, fake, null, 64, 768, 16, fake, fake,
                                             fake + 8, null) == -5
    bws = lib.parrot_experts_workspace_bytes(4096, 768, 512, 256)
    blocks = lambda **kw: lib.parrot_experts_gate_up_grouping_blocks_bf16(*[
        kw.get(k, v) for k, v in (
            ("x", fake), ("T", 4096), ("dim", 768), ("E", 32), ("H", 512), ("Hs", 256),
            ("C", 512), ("tab", fake), ("cnt", fake), ("off", fake), ("srt", fake),
            ("gu", fake), ("sgu", fake), ("ws", fake), ("wsb", bws), ("stream", null))])
    assert blocks(tab=null) == -1 and blocks(srt=null) == -1
    assert blocks(T=4097, wsb=lib.parrot_experts_workspace_bytes(4097, 768, 512, 256)) == -3
    assert blocks(E=16, C=1024) == -3  # wide tiles at 512 rows per expert
    assert blocks(tab=fake + 8) == -5
    # the ids form stays within its own shapes
    assert lib.parrot_experts_gate_up_grouping_bf16(
        fake, 4096, 768, 32, 512, 256, 512, fake, fake, fake, fake, fake, fake, fake, bws,
        null) == -3
    gws = lib.parrot_experts_workspace_bytes(512, 768, 512, 256)
    assert lib.parrot_experts_gate_up_grouping_bf16(
        fake, 512, 768, 16, 512, 256, 80, null, fake, fake, fake, fake, fake, fake, gws,
        null) == -1
    assert lib.parrot_experts_gate_up_grouping_bf16(
        fake, 2048, 768, 16, 512, 256, 264, fake, fake, fake, fake, fake, fake, fake,
        lib.parrot_experts_workspace_bytes(2048, 768, 512, 256), null) == -3
    assert lib.parrot_experts_gate_up_grouping_bf16(
        fake, 512, 768, 16, 512, 256, 80, fake, fake, fake, fake, fake, fake, fake, 16,
        null) == -4
    assert lib.parrot_experts_down_sorted_bf16(
        512, 768, 16, 512, 256, 80, fake, fake, null, fake, fake, fake, fake, gws, null) == -1
    assert lib.parrot_experts_down_sorted_bf16(
        512, 96, 16, 512, 256, 80, fake, fake, fake, fake, fake, fake, fake, gws, null) == -3


def test_static_scratch_entry_rejects_before_any_hip_call(lib):
    """The allocation-free grouped experts entry states its limit in the
    header and refuses larger inputs (and bad shapes) on the host."""
    from parrot import _abi
    header = HEADER.read_text()
    assert "#define PARROT_STATIC_SCRATCH_BYTES ((size_t)30 << 20)" in header
    assert _abi.STATIC_SCRATCH_BYTES == 30 << 20
    fn = lib.parrot_grouped_experts_static_bf16
    null = [None] * 11
    # 4096 tokens at the default shapes fill the array exactly; 4097 do not fit.
    assert lib.parrot_experts_workspace_bytes(4096, 768, 512, 256) == _abi.STATIC_SCRATCH_BYTES
    assert fn(None, 4097, 768, 16, 512, 256, 1032, *null, None) == -6
    assert fn(None, 100, 0, 16, 512, 256, 32, *null, None) == -2
    assert fn(None, -1, 768, 16, 512, 256, 32, *null, None) == -2
