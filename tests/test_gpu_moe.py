"""GPU parity of the bandwidth kernels and the grouped MoE layer.

Tolerance: bf16 outputs within max-abs 2e-2 and
mean-abs 2e-3 of the fp32 oracle evaluated on the same (bf16-valued)
inputs and weights.  The RMSNorm / depth-mix kernels round once, so they are
also held to one bf16 ulp of the oracle's value.
"""
import numpy as np
import pytest
import torch

from moe_cases import MAX_ABS, MEAN_ABS, error_stats, inputs, moe_module, oracle_moe, skew_bias
from oracle import layers

pytestmark = pytest.mark.gpu



def _say(msg):
    print(msg, flush=True)


def _ulp_ok(got: torch.Tensor, ref: torch.Tensor, scale: torch.Tensor | None = None):
    """One bf16 rounding of a value within fp32 reassociation error of the
    oracle: |got - ref| <= ulp_bf16(ref) + 1e-5 * scale + 1e-6, where scale
    is the magnitude of the summands (|ref| unless given)."""
    ref = ref.detach().float().cpu()
    got = got.detach().float().cpu()
    scale = ref.abs() if scale is None else scale.detach().float().cpu()
    ulp = torch.ldexp(torch.ones_like(ref), torch.frexp(ref)[1] - 8)
    excess = (got - ref).abs() - (ulp + 1e-5 * scale + 1e-6)
    assert (excess <= 0).all(), float(excess.max())


class _Norm(torch.nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = torch.nn.Parameter((torch.rand(dim) + 0.5))
        self.eps = eps


@pytest.mark.parametrize("rows,dim", [(1, 768), (7, 768), (512, 768), (4097, 768), (33, 64),
                                      (16, 2048), (5, 4096)])
def test_rms_norm(rows, dim):
    from parrot import hip_moe
    _say(f"rms_norm rows={rows} dim={dim}")
    norm = _Norm(dim).cuda().bfloat16()
    x = (torch.randn(rows, dim) * 3).cuda().bfloat16()
    with torch.no_grad():
        got = hip_moe.rms_norm(norm, x)
    ref = layers.rms_norm(x.float().cpu(), norm.weight.float().cpu(), 1e-6)
    _ulp_ok(got, ref)


class _Depth(torch.nn.Module):
    def __init__(self, dim):
        super().__init__()
        self.query = torch.nn.Parameter(torch.randn(dim) * 0.5)
        self.norm = _Norm(dim)


@pytest.mark.parametrize("sources", [1, 2, 5, 9])
@pytest.mark.parametrize("tokens,dim", [(1, 768), (16, 768), (512, 768), (100, 64), (3, 2048)])
def test_depth_mix_and_norm(sources, tokens, dim):
    from parrot import hip_moe
    _say(f"depth_mix S={sources} T={tokens} dim={dim}")
    torch.manual_seed(sources * 100 + tokens)
    depth = _Depth(dim).cuda().bfloat16()
    out_norm = _Norm(dim).cuda().bfloat16()
    src = [(torch.randn(tokens, dim) * (1 + s)).cuda().bfloat16() for s in range(sources)]
    with torch.no_grad():
        mix = hip_moe.depth_mix(depth, src)
        fused = hip_moe.depth_mix_norm(depth, src, out_norm)
    cpu = [s.float().cpu() for s in src]
    ref = layers.depth_mix(cpu, depth.query.float().cpu(), depth.norm.weight.float().cpu(), 1e-6)
    _ulp_ok(mix, ref, scale=torch.stack(cpu).abs().amax(0))
    # fused: the norm consumes the bf16-rounded mix, exactly as unfused
    ref_norm = layers.rms_norm(mix.float().cpu(), out_norm.weight.float().cpu(), 1e-6)
    _ulp_ok(fused, ref_norm)


@pytest.mark.parametrize("sources,dim", [(9, 768), (2, 768), (5, 1024), (3, 64), (1, 448)])
def test_depth_mix_wave_kernel_equals_token_kernel(sources, dim):
    """From 4096 tokens the depth mix runs one wavefront per token
    (depth_mix_wave_kernel) instead of one workgroup per token: every token's
    mix and normalised mix are the same bits either way (the same products,
    DPP reductions and slice order), so a token's result does not depend on
    the batch it is in.  Checked by mixing 5,000 tokens at once against the
    same rows mixed in chunks below the threshold."""
    from parrot import hip_moe
    _say(f"depth mix wave kernel S={sources} dim={dim}")
    torch.manual_seed(sources * 7 + dim)
    depth = _Depth(dim).cuda().bfloat16()
    out_norm = _Norm(dim).cuda().bfloat16()
    tokens = 5000
    src = [(torch.randn(tokens, dim) * (1 + s)).cuda().bfloat16() for s in range(sources)]
    with torch.no_grad():
        mix = hip_moe.depth_mix(depth, src)
        fused = hip_moe.depth_mix_norm(depth, src, out_norm)
        parts = [(0, 1), (1, 1000), (1000, 3000), (3000, 5000)]
        mix_ref = torch.cat([hip_moe.depth_mix(depth, [x[a:b] for x in src]) for a, b in parts])
        fused_ref = torch.cat([hip_moe.depth_mix_norm(depth, [x[a:b] for x in src], out_norm)
                               for a, b in parts])
    assert torch.equal(mix, mix_ref)
    assert torch.equal(fused, fused_ref)
    cpu = [x.float().cpu() for x in src]
    ref = layers.depth_mix(cpu, depth.query.float().cpu(), depth.norm.weight.float().cpu(), 1e-6)
    _ulp_ok(mix, ref, scale=torch.stack(cpu).abs().amax(0))


MOE_CASES = [
    ("C2", 256, 32, False),
    ("C3", 4096, 32, True),
    ("C4", 512, 16, False),
    ("C5_b1", 1, 16, False),
    ("C5_b2", 2, 16, False),
    ("C5_b8", 8, 16, False),
    ("odd", 130, 16, False),
    ("large", 16384, 16, False),
    # 4,096 rows per expert: down on 256 x 256 tiles (gate/up on 128 x 128)
    ("wide256", 8192, 4, False),
    ("wide256_skew", 8192, 4, True),
]


@pytest.mark.parametrize("tokens,dim", [(1, 768), (17, 768), (512, 768), (5000, 768), (40, 448)])
def test_embed_depth_mix_equals_gather_and_mix(tokens, dim):
    """The forward's first launch (parrot_embed_depth_mix_bf16): the gathered
    embedding rows equal table[ids] and the first module's input equals the
    separate depth_mix_norm of that one source, bit for bit (from 4096 tokens
    the separate mix runs the one-wavefront kernel); ids outside the table
    read its nearest row; the stat buffer is zero-filled, also with no
    tokens."""
    from parrot import hip_moe
    _say(f"embed + first depth mix T={tokens} dim={dim}")
    torch.manual_seed(tokens + dim)
    vocab = 1000
    depth = _Depth(dim).cuda().bfloat16()
    with torch.no_grad():
        depth.query.normal_()
    out_norm = _Norm(dim).cuda().bfloat16()
    table = (torch.randn(vocab, dim) * 2).cuda().bfloat16()
    ids = torch.randint(0, vocab, (1, tokens)).cuda()
    ids[0, 0] = -5
    ids[0, -1] = vocab + 3
    zeros = torch.full((257,), float("nan"), device="cuda")
    with torch.no_grad():
        rows, first = hip_moe.embed_depth_mix_norm(ids, table, depth, out_norm, zeros)
        clamped = ids.clamp(0, vocab - 1)
        ref_rows = table[clamped]
        ref_first = hip_moe.depth_mix_norm(depth, [ref_rows], out_norm)
    assert torch.equal(rows, ref_rows)
    assert torch.equal(first, ref_first)
    assert torch.equal(zeros, torch.zeros_like(zeros))
    empty = torch.full((5,), float("nan"), device="cuda")
    with torch.no_grad():
        hip_moe.embed_depth_mix_norm(ids[:, :0], table, depth, out_norm, empty)
    torch.cuda.synchronize()
    assert torch.equal(empty, torch.zeros_like(empty))


@pytest.mark.parametrize("name,tokens,experts,skewed", MOE_CASES)
def test_moe_layer(name, tokens, experts, skewed):
    from parrot import hip_moe
    _say(f"moe layer {name}: T={tokens} E={experts} skew={skewed}")
    module = moe_module(experts, seed=1)
    x = inputs(tokens, seed=1 + tokens)
    bias = skew_bias(experts) if skewed else None
    with torch.no_grad():
        routed = hip_moe.route(module, x, False, logit_bias=bias)
        out = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                          grouping=routed.grouping)
    idx = routed.indices.cpu().numpy()
    ref, ref_idx, _, _ = oracle_moe(module, x, logit_bias=None if bias is None else bias.numpy())
    same = (ref_idx == idx).all(-1)
    _say(f"  routing agreement {same.mean():.5f}; overflow "
         f"{int(routed.grouping.offsets[-1])} of {2 * tokens}")
    assert same.mean() >= 0.995
    # Compare every token with the oracle evaluated on the HIP's routing.
    ref_same, _, _, _ = oracle_moe(module, x, indices=idx, weights=routed.weights.cpu().numpy())
    mx, mean = error_stats(out, ref_same)
    _say(f"  max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx <= MAX_ABS and mean <= MEAN_ABS
    mx2, mean2 = error_stats(out[torch.from_numpy(same).cuda()], ref[torch.from_numpy(same)])
    assert mx2 <= MAX_ABS and mean2 <= MEAN_ABS


@pytest.mark.parametrize("tokens,experts,dim,hidden,shared", [
    (40, 8, 1024, 1280, 256),     # small-T plan with K > 768: pipelined 32-row tiles
    (1200, 8, 1024, 1280, 256),   # many rows per expert, K > 768: pipelined 32-row tiles
    (300, 4, 2048, 512, 192),     # widest supported dim
])
def test_moe_layer_other_widths(tokens, experts, dim, hidden, shared):
    from parrot import hip_moe
    _say(f"moe layer T={tokens} E={experts} dim={dim} H={hidden} Hs={shared}")
    module = moe_module(experts, seed=7, dim=dim, hidden=hidden, shared=shared)
    x = inputs(tokens, seed=7, dim=dim)
    with torch.no_grad():
        routed = hip_moe.route(module, x, False)
        out = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                          grouping=routed.grouping)
    ref, _, _, _ = oracle_moe(module, x, indices=routed.indices.cpu().numpy(),
                              weights=routed.weights.cpu().numpy())
    mx, mean = error_stats(out, ref)
    _say(f"  max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx <= MAX_ABS and mean <= MEAN_ABS


def test_moe_addend_and_tiny_shapes():
    from parrot import hip_moe
    _say("moe addend + tiny widths")
    module = moe_module(8, seed=4, dim=64, hidden=128, shared=64)
    x = inputs(64, seed=4, dim=64)
    addend = inputs(64, seed=5, dim=64)
    with torch.no_grad():
        routed = hip_moe.route(module, x, False)
        out = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                          addend=addend, grouping=routed.grouping)
        delta = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                            grouping=routed.grouping)
    # identical rounding sequence to `addend + delta` in bf16
    assert torch.equal(out, addend + delta)
    ref, _, _, _ = oracle_moe(module, x, indices=routed.indices.cpu().numpy(),
                              weights=routed.weights.cpu().numpy())
    mx, mean = error_stats(delta, ref)
    assert mx <= MAX_ABS and mean <= MEAN_ABS


def test_experts_from_external_indices():
    """grouped_hip_experts without a HIP route (positions recomputed)."""
    from parrot import hip_moe
    _say("experts from external indices")
    module = moe_module(16, seed=6)
    x = inputs(300, seed=6)
    rng = np.random.default_rng(6)
    idx = np.stack([rng.choice(16, 2, replace=False) for _ in range(300)]).astype(np.int64)
    idx[:200, 0] = 3  # heavy skew onto expert 3 -> overflow
    idx[:200, 1] = np.where(idx[:200, 1] == 3, 4, idx[:200, 1])
    w = rng.random((300, 2)).astype(np.float32)
    with torch.no_grad():
        out = hip_moe.grouped_hip_experts(module, x, torch.from_numpy(idx).cuda(),
                                          torch.from_numpy(w).cuda())
    ref, _, _, _ = oracle_moe(module, x, indices=idx, weights=w)
    mx, mean = error_stats(out, ref)
    assert mx <= MAX_ABS and mean <= MEAN_ABS


@pytest.mark.parametrize("b,t,start,expand", [(1, 512, 0, True), (2, 37, 5, False), (3, 1, 4000, False)])
def test_rope_qkv(b, t, start, expand):
    """RoPE + head split vs the oracle's fp32 rotation (parrot/model.py:206-230)."""
    from types import SimpleNamespace

    from oracle import parrot_fp32
    from parrot import hip_moe
    from parrot.model import ModelConfig, _rope_tables
    _say(f"rope b={b} t={t} start={start} expand={expand}")
    c = ModelConfig()
    H, Hk, d = c.n_heads, c.n_kv_heads, c.head_dim
    qkv = (torch.randn(b, t, (H + 2 * Hk) * d) * 2).cuda().bfloat16()
    cos, sin = _rope_tables(c, torch.empty(0, device="cuda"))
    with torch.no_grad():
        q, k, v = hip_moe.rope_qkv(qkv, cos, sin, H, Hk, d, start, expand)
    # The rotation is checked in fp32 against the kernel's own angle tables;
    # the tables themselves are checked against the oracle's formula below.
    x = qkv.float().cpu()
    heads = x.view(b, t, H + 2 * Hk, d).transpose(1, 2)
    c_t, s_t = cos.cpu()[start:start + t], sin.cpu()[start:start + t]

    def rotate(h):
        out = torch.empty_like(h)
        even, odd = h[..., 0::2], h[..., 1::2]
        out[..., 0::2] = even * c_t - odd * s_t
        out[..., 1::2] = even * s_t + odd * c_t
        return out

    ref_q = rotate(heads[:, :H])
    ref_k = rotate(heads[:, H:H + Hk])
    ref_v = heads[:, H + Hk:]
    oracle = parrot_fp32.ParrotFP32(SimpleNamespace(rope_theta=c.rope_theta, head_dim=d), {})
    ones = torch.zeros(1, 1, t, d)
    ones[..., 0::2] = 1.0
    table = oracle._rope(ones, start)  # rotating (1, 0) pairs yields (cos, sin)
    assert (table[0, 0, :, 0::2] - c_t).abs().max() < 2e-3
    assert (table[0, 0, :, 1::2] - s_t).abs().max() < 2e-3
    rep = H // Hk if expand else 1
    _ulp_ok(q, ref_q)
    _ulp_ok(k, ref_k.repeat_interleave(rep, dim=1))
    assert torch.equal(v.float().cpu(), ref_v.repeat_interleave(rep, dim=1))
    if not expand:  # transposed values for the attention kernel, same q and k
        with torch.no_grad():
            q2, k2, vt = hip_moe.rope_qkv(qkv, cos, sin, H, Hk, d, start, False,
                                          vt_keys=hip_moe.padded_keys(t))
        assert torch.equal(q2, q) and torch.equal(k2, k)
        assert vt.shape == (b, Hk, d, hip_moe.padded_keys(t))
        assert torch.equal(vt[..., :t].transpose(-1, -2), v)


@pytest.mark.parametrize("tokens,n_older", [(512, 3), (130, 0), (64, 8), (17, 1)])
def test_combine_then_depth_mix(tokens, n_older):
    """The combine folded into the next module's depth mix writes exactly the
    combine's output and exactly the depth mix + norm of it with the older
    sources (the same kernel arithmetic, the new row taken from registers)."""
    from moe_cases import inputs, moe_module
    from parrot import hip_moe
    _say(f"combine + depth mix T={tokens} older={n_older}")
    module = moe_module(16, seed=3)
    x = inputs(tokens, seed=4)
    addend = inputs(tokens, seed=5)
    depth = _Depth(x.shape[1]).cuda().bfloat16()
    norm = _Norm(x.shape[1]).cuda().bfloat16()
    older = [inputs(tokens, seed=10 + i) * (1 + i) for i in range(n_older)]
    with torch.no_grad():
        routed = hip_moe.route(module, x, False)
        plain = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                            addend=addend, grouping=routed.grouping)
        fused, mixed = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                                   addend=addend, grouping=routed.grouping,
                                                   then_mix=(depth, older, norm))
        ref = hip_moe.depth_mix_norm(depth, older + [plain], norm)
    assert torch.equal(fused, plain)
    assert torch.equal(mixed, ref)


@pytest.mark.parametrize("tokens,experts,sources,skewed", [
    (512, 16, 5, False), (17, 16, 1, False), (256, 32, 9, False), (1000, 32, 3, True),
    (100, 8, 2, False), (4097, 16, 4, False)])
def test_depth_mix_route(tokens, experts, sources, skewed):
    """The depth mix that also routes its normalised output writes exactly
    depth_mix_norm's rows and exactly route()'s weights and indices on them
    (the same MFMA logit chains, token in A row 0)."""
    from parrot import hip_moe
    _say(f"depth mix + route T={tokens} E={experts} S={sources} skew={skewed}")
    module = moe_module(experts, seed=2)
    depth = _Depth(768).cuda().bfloat16()
    norm = _Norm(768).cuda().bfloat16()
    src = [inputs(tokens, seed=20 + s) * (1 + s) for s in range(sources)]
    bias = skew_bias(experts) if skewed else None
    with torch.no_grad():
        normed, top2 = hip_moe.depth_mix_norm_route(depth, src, norm, module, logit_bias=bias)
        ref = hip_moe.depth_mix_norm(depth, src, norm)
        routed = hip_moe.route(module, ref, False, logit_bias=bias)
    assert torch.equal(normed, ref)
    assert torch.equal(top2.indices, routed.indices)
    assert torch.equal(top2.weights, routed.weights)


def _sorted_from_grouping(g, experts):
    """Assignment id of each hidden row: expert-contiguous slot order, the
    in-capacity slots perm[e, :] then the expert's overflow entries."""
    counts = g.counts.cpu().tolist()
    offsets = g.offsets.cpu().tolist()
    perm = g.perm.cpu()
    overflow = g.overflow.cpu()
    rows = []
    for e in range(experts):
        inside = min(counts[e], g.capacity)
        rows += perm[e, :inside].tolist()
        start = offsets[experts + 1 + e]
        rows += overflow[start:start + counts[e] - inside].tolist()
    return torch.tensor(rows, dtype=torch.int32)


@pytest.mark.parametrize("tokens,experts,skewed", [
    (512, 16, False), (300, 16, True), (17, 16, False), (1000, 32, True), (100, 8, False),
    (1024, 32, False)])
def test_experts_group_in_kernel(tokens, experts, skewed):
    """The gate/up launch that groups the top-2 ids itself gives the same
    MoE output as the route + group path, and the grouping it writes (counts,
    offsets, the hidden rows' assignment ids) is that path's grouping."""
    from parrot import hip_moe
    _say(f"in-kernel grouping T={tokens} E={experts} skew={skewed}")
    module = moe_module(experts, seed=8)
    x = inputs(tokens, seed=8)
    assert hip_moe.groups_in_kernel(module, tokens, x.shape[1])
    bias = skew_bias(experts) if skewed else None
    addend = inputs(tokens, seed=9)
    with torch.no_grad():
        routed = hip_moe.route(module, x, False, logit_bias=bias)
        ref = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                          addend=addend, grouping=routed.grouping)
        got = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                          addend=addend)
    g = routed.grouping
    _say(f"  overflow {int(g.offsets[-1])} of {2 * tokens}")
    assert torch.equal(got, ref)
    buf = module.__dict__["_hip_group_buffers"][:4 * (3 * experts + 2 + 2 * tokens)]
    buf = buf.view(torch.int32).cpu()
    assert torch.equal(buf[:experts], g.counts.cpu())
    assert torch.equal(buf[experts:3 * experts + 2], g.offsets.cpu())
    assert torch.equal(buf[3 * experts + 2:], _sorted_from_grouping(g, experts))


@pytest.mark.parametrize("tokens,experts,skewed", [
    (4096, 32, True), (2048, 16, False), (1025, 32, False), (300, 16, True), (17, 16, False),
    (4096, 32, False)])
def test_experts_group_from_route_blocks(tokens, experts, skewed):
    """The gate/up launch that groups from the route block table (the form
    past 2048 assignments; it also takes the smaller shapes) gives the route +
    group path's MoE output bit for bit, and writes that path's grouping
    (counts, offsets, the hidden rows' assignment ids); through the C-ABI
    entries as the standalone layer calls them."""
    from parrot import _abi, hip_moe
    from parrot._abi import ptr
    _say(f"grouping from the route block table T={tokens} E={experts} skew={skewed}")
    module = moe_module(experts, seed=10)
    x = inputs(tokens, seed=10)
    cfg = module.cfg
    dim, H, Hs = x.shape[1], cfg.expert_dim, cfg.shared_expert_dim
    lib = _abi.load()
    assert lib.parrot_experts_group_in_kernel(tokens, dim, experts, H, Hs) in (1, 2)
    bias = skew_bias(experts) if skewed else None
    with torch.no_grad():
        routed = hip_moe.route(module, x, False, logit_bias=bias)
        ref = hip_moe.grouped_hip_experts(module, x, routed.indices, routed.weights,
                                          grouping=routed.grouping)
        tab = hip_moe.route_top2(module, x, logit_bias=bias, blocks=True)
    assert torch.equal(tab.indices, routed.indices) and torch.equal(tab.weights, routed.weights)
    g = routed.grouping
    _say(f"  overflow {int(g.offsets[-1])} of {2 * tokens}, max count {int(g.counts.max())}")
    gate_up, down, shared_gate_up, shared_down = hip_moe.pack_expert_weights(module)
    nbytes = lib.parrot_experts_workspace_bytes(tokens, dim, H, Hs)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    i32 = dict(dtype=torch.int32, device="cuda")
    counts, offsets = torch.empty(experts, **i32), torch.empty(2 * experts + 2, **i32)
    sorted_ids = torch.empty(2 * tokens, **i32)
    out = torch.empty_like(x)
    cap = hip_moe.capacity(tokens, experts)
    s = torch.cuda.current_stream().cuda_stream
    _abi.check(lib.parrot_experts_gate_up_grouping_blocks_bf16(
        ptr(x), tokens, dim, experts, H, Hs, cap, ptr(tab.blocks), ptr(counts), ptr(offsets),
        ptr(sorted_ids), ptr(gate_up), ptr(shared_gate_up), ptr(ws), nbytes, s), "gate/up")
    _abi.check(lib.parrot_experts_down_sorted_bf16(
        tokens, dim, experts, H, Hs, cap, ptr(counts), ptr(offsets), ptr(sorted_ids),
        ptr(tab.weights), ptr(down), ptr(shared_down), ptr(ws), nbytes, s), "down")
    _abi.check(lib.parrot_experts_combine_bf16(tokens, dim, H, Hs, None, ptr(out), ptr(ws),
                                               nbytes, s), "combine")
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(counts.cpu(), g.counts.cpu())
    assert torch.equal(offsets.cpu(), g.offsets.cpu())
    assert torch.equal(sorted_ids.cpu(), _sorted_from_grouping(g, experts))


@pytest.mark.parametrize("tokens,experts,older,with_base", [
    (512, 16, 2, True), (512, 16, 1, False), (17, 32, 8, True), (1000, 16, 4, True)])
def test_depth_mix_route_pending(tokens, experts, older, with_base):
    """The MoE input mix with a deferred attention output as its last
    source: `resolved` is bf16(base + bf16(sum of the 8 heads' fp32
    contributions in head order)) bit for bit (restated on the host), and
    the normalised rows, weights and indices equal depth_mix_norm_route's on
    the explicit sources older + [resolved]."""
    from parrot import hip_moe
    _say(f"depth mix + route, pending T={tokens} E={experts} older={older} base={with_base}")
    module = moe_module(experts, seed=6)
    depth = _Depth(768).cuda().bfloat16()
    norm = _Norm(768).cuda().bfloat16()
    src = [inputs(tokens, seed=40 + s) * (1 + s) for s in range(older)]
    g = torch.Generator().manual_seed(tokens + older)
    contrib = (torch.randn(tokens, 8, 768, generator=g) * 0.05).float()
    # head sums of exactly -0 and +0 (a missing base must keep their signs)
    contrib[0] = -0.0
    contrib[1, :, :384] = 0.0
    base = inputs(tokens, seed=60) if with_base else None
    # host restatement: fp32 sum in head order, bf16, then bf16(base + that)
    acc = contrib[:, 0].clone()
    for h in range(1, 8):
        acc = acc + contrib[:, h]
    want = acc.bfloat16()
    if base is not None:
        want = (base.cpu().float() + want.float()).bfloat16()
    with torch.no_grad():
        resolved = torch.empty_like(src[0])
        placeholder = base if base is not None else src[0]
        normed, top2 = hip_moe.depth_mix_norm_route(
            depth, src + [placeholder], norm, module,
            pending=(contrib.cuda(), base, resolved))
        ref, ref_top2 = hip_moe.depth_mix_norm_route(depth, src + [want.cuda()], norm, module)
    assert torch.equal(resolved.cpu().view(torch.int16), want.view(torch.int16))  # bits
    assert torch.equal(normed, ref)
    assert torch.equal(top2.indices, ref_top2.indices)
    assert torch.equal(top2.weights, ref_top2.weights)
