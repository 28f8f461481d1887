"""GPU parity of the decode-step attention kernels and of graph-replayed
decoding.

The kernels are checked against a plain fp32 CPU restatement of the
reference decode attention (parrot/model.py:239-262 for the sliding-window
GQA layers, 399-432 for MLA over the latent cache) on random caches, at
positions below, at and past the window, including the cache update.  The
captured decode step must reproduce eager decoding bit for bit.
"""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _attend(q, keys, values, scale):
    """fp32 softmax(q k^T scale) v; q [H, d], keys/values [L, d] per head."""
    s = (q @ keys.T) * scale
    return torch.softmax(s, dim=-1) @ values


@pytest.mark.parametrize("position", [0, 5, 63, 64, 200])
def test_decode_attention_window(position):
    from parrot import hip_moe
    b, H, Hk, d, max_pos, window = 3, 8, 2, 96, 256, 64
    _say(f"decode attention p={position} window={window}")
    g = torch.Generator().manual_seed(position)
    kc = torch.randn(b, Hk, max_pos, d, generator=g).bfloat16()
    vc = torch.randn(b, Hk, max_pos, d, generator=g).bfloat16()
    q = torch.randn(b, H, 1, d, generator=g).bfloat16()
    kn = torch.randn(b, Hk, 1, d, generator=g).bfloat16()
    vn = torch.randn(b, Hk, 1, d, generator=g).bfloat16()
    kc_g, vc_g = kc.cuda(), vc.cuda()
    pos = torch.tensor([position], dtype=torch.int32, device="cuda")
    with torch.no_grad():
        out = hip_moe.decode_attention(q.cuda(), kn.cuda(), vn.cuda(), kc_g, vc_g, pos, window,
                                       d ** -0.5)
    # cache: row `position` replaced, every other row untouched
    kc_ref, vc_ref = kc.clone(), vc.clone()
    kc_ref[:, :, position] = kn[:, :, 0]
    vc_ref[:, :, position] = vn[:, :, 0]
    assert torch.equal(kc_g.cpu(), kc_ref) and torch.equal(vc_g.cpu(), vc_ref)
    lo = max(0, position - window + 1)
    ref = torch.empty(b, H, d)
    for bi in range(b):
        for h in range(H):
            kv = h // (H // Hk)
            ref[bi, h] = _attend(q[bi, h].float(), kc_ref[bi, kv, lo:position + 1].float(),
                                 vc_ref[bi, kv, lo:position + 1].float(), d ** -0.5)
    got = out.float().cpu().view(b, H, d)
    # one bf16 rounding of the output plus fp32 reassociation
    assert (got - ref).abs().max() <= 2 ** -8 * ref.abs().max() + 1e-5


@pytest.mark.parametrize("batch,position", [(1, 0), (2, 63), (1, 200), (3, 64), (4, 150)])
def test_decode_attention_heads(batch, position):
    """The deferred form: the same cache update as decode_attention, and
    per-head contributions equal to the products of decode_attention's own
    bf16 output with each head's slice of the output projection (fp64 on
    the CPU, fp32 reassociation tolerance).  Summed over heads, rounded and
    added to an addend they match the undeferred projection within one bf16
    rounding of each sum."""
    from parrot import hip_moe
    H, Hk, d, max_pos, window, dim = 8, 2, 96, 256, 64, 768
    _say(f"decode attention heads b={batch} p={position}")
    g = torch.Generator().manual_seed(100 + position + batch)
    kc = torch.randn(batch, Hk, max_pos, d, generator=g).bfloat16()
    vc = torch.randn(batch, Hk, max_pos, d, generator=g).bfloat16()
    q = torch.randn(batch, H, 1, d, generator=g).bfloat16().cuda()
    kn = torch.randn(batch, Hk, 1, d, generator=g).bfloat16().cuda()
    vn = torch.randn(batch, Hk, 1, d, generator=g).bfloat16().cuda()
    wo = (torch.randn(dim, H * d, generator=g) * (H * d) ** -0.5).bfloat16().cuda()
    addend = torch.randn(batch, 1, dim, generator=g).bfloat16().cuda()
    pos = torch.tensor([position], dtype=torch.int32, device="cuda")
    kc_a, vc_a, kc_b, vc_b = kc.cuda(), vc.cuda(), kc.cuda(), vc.cuda()
    with torch.no_grad():
        y = hip_moe.decode_attention(q, kn, vn, kc_a, vc_a, pos, window, d ** -0.5)
        contrib = hip_moe.decode_attention_heads(q, kn, vn, kc_b, vc_b, pos, window, d ** -0.5,
                                                 wo)
        undeferred = hip_moe.decode_linear(y.view(batch, 1, H * d), wo, addend)
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)
    assert contrib.shape == (batch, H, dim) and contrib.dtype == torch.float32
    yd = y.double().cpu().view(batch, H, d)
    w = wo.double().cpu().view(dim, H, d)
    ref = torch.einsum("bhi,nhi->bhn", yd, w)
    scale = torch.einsum("bhi,nhi->bhn", yd.abs(), w.abs())
    assert ((contrib.double().cpu() - ref).abs() <= 1e-6 * scale + 1e-7).all()
    # The resolved module output against the undeferred GEMV + addend.
    acc = contrib[:, 0].clone()
    for h in range(1, H):
        acc = acc + contrib[:, h]
    resolved = (addend.float().view(batch, dim) + acc.bfloat16().float()).bfloat16()
    got, want = resolved.float().cpu(), undeferred.float().cpu().view(batch, dim)
    tol = 2 ** -7 * (addend.float().cpu().view(batch, dim).abs() + 2 * acc.abs().cpu()) + 1e-6
    assert ((got - want).abs() <= tol).all()


@pytest.mark.parametrize("tokens,lanes,with_base,sources", [
    (1, 8, True, 3), (2, 8, False, 1), (5, 11, True, 9), (16, 1, True, 4)])
def test_decode_moe_resolves_a_pending_source(tokens, lanes, with_base, sources):
    """A pending last depth source resolved inside the decode MoE's input
    mix: the resolved rows equal bf16(base + bf16(the lanes summed in order))
    computed on the CPU, and the MoE's outputs equal those of the same launch
    given the resolved rows as an ordinary source, bit for bit."""
    from moe_cases import inputs, moe_module
    from test_gpu_moe import _Depth, _Norm
    from parrot import hip_moe
    _say(f"decode moe pending T={tokens} lanes={lanes} base={with_base} S={sources}")
    torch.manual_seed(40 + tokens + lanes)
    module = moe_module(16, seed=17)
    depth = _Depth(768).cuda().bfloat16()
    norm = _Norm(768).cuda().bfloat16()
    src = [inputs(tokens, seed=50 + s).view(tokens, 1, 768) * (1 + s) for s in range(sources - 1)]
    g = torch.Generator().manual_seed(60 + tokens)
    contrib = (torch.randn(tokens, lanes, 768, generator=g) * 0.3).cuda()
    base = inputs(tokens, seed=61).view(tokens, 1, 768) if with_base else None
    acc = torch.zeros(tokens, 768)
    for l in range(lanes):
        acc = acc + contrib[:, l].cpu()
    ref = acc.bfloat16()
    if base is not None:
        ref = (base.cpu().float().view(tokens, 768) + ref.float()).bfloat16()
    ref = ref.view(tokens, 1, 768).cuda()
    placeholder = base if base is not None else (src[0] if src else ref)
    with torch.no_grad():
        resolved = torch.empty(tokens, 1, 768, dtype=torch.bfloat16, device="cuda")
        out, idx, w = hip_moe.decode_experts(
            module, None, addend=resolved, mix=(depth, src + [placeholder], norm),
            pending=(contrib, base, resolved))
        out2, idx2, w2 = hip_moe.decode_experts(module, None, addend=ref,
                                                mix=(depth, src + [ref], norm))
    assert torch.equal(resolved, ref)
    assert torch.equal(idx, idx2) and torch.equal(w, w2) and torch.equal(out, out2)


@pytest.mark.parametrize("position", [0, 150, 299])
def test_decode_attention_latent(position):
    from parrot import hip_moe
    b, H, r, max_pos = 2, 8, 128, 300
    _say(f"latent decode attention p={position}")
    g = torch.Generator().manual_seed(100 + position)
    lat = torch.randn(b, max_pos, r, generator=g).bfloat16()
    new = torch.randn(b, 1, r, generator=g).bfloat16()
    q = torch.randn(b, 1, H * r, generator=g)
    lat_g = lat.cuda()
    pos = torch.tensor([position], dtype=torch.int32, device="cuda")
    scale = 96 ** -0.5
    with torch.no_grad():
        out = hip_moe.decode_attention_latent(q.cuda(), new.cuda(), lat_g, pos, H, scale)
    lat_ref = lat.clone()
    lat_ref[:, position] = new[:, 0]
    assert torch.equal(lat_g.cpu(), lat_ref)
    ref = torch.empty(b, H, r)
    for bi in range(b):
        keys = lat_ref[bi, :position + 1].float()
        for h in range(H):
            ref[bi, h] = _attend(q[bi, 0, h * r:(h + 1) * r], keys, keys, scale)
    got = out.cpu().view(b, H, r)
    assert (got - ref).abs().max() <= 1e-4 * ref.abs().max() + 1e-5


@pytest.mark.parametrize("tokens,with_addend", [(1, True), (3, False), (8, True), (16, True)])
def test_mla_decode_projections(tokens, with_addend):
    """The MLA decode projections around the latent attention against fp32 CPU
    products of the same bf16 weights (parrot/model.py:417-431)."""
    from parrot import hip_moe
    dim, heads, r = 768, 8, 128
    width = heads * r
    _say(f"mla decode projections T={tokens} addend={with_addend}")
    g = torch.Generator().manual_seed(40 + tokens)
    x = torch.randn(tokens, 1, dim, generator=g).bfloat16()
    wq = (torch.randn(width, dim, generator=g) * 0.05).bfloat16()
    wkv = (torch.randn(r, dim, generator=g) * 0.05).bfloat16()
    wo = (torch.randn(dim, width, generator=g) * 0.05).bfloat16()
    ctx = torch.randn(tokens, width, generator=g)
    addend = torch.randn(tokens, 1, dim, generator=g).bfloat16() if with_addend else None
    with torch.no_grad():
        q, lat = hip_moe.mla_decode_in(x.cuda(), wq.cuda(), wkv.cuda())
        out = hip_moe.mla_decode_out(ctx.cuda(), wo.cuda(),
                                     None if addend is None else addend.cuda())
    assert q.shape == (tokens, width) and q.dtype == torch.float32
    assert lat.shape == (tokens, 1, r) and lat.dtype == torch.bfloat16
    assert out.shape == (tokens, 1, dim) and out.dtype == torch.bfloat16
    xf = x.float().view(tokens, dim)
    # fp32 sums of exact products: only the order of additions differs
    q_ref = xf @ wq.float().T
    bound = 1e-5 * (xf.abs() @ wq.float().abs().T) + 1e-6
    assert ((q.cpu() - q_ref).abs() <= bound).all()
    # one bf16 rounding of an fp32 sum: at most one bf16 step apart
    lat_ref = (xf @ wkv.float().T).view(tokens, 1, r)
    assert ((lat.cpu().float() - lat_ref).abs() <= 2 ** -7 * lat_ref.abs() + 1e-6).all()
    res_ref = (ctx @ wo.float().T).view(tokens, 1, dim)
    if addend is None:
        ref, tol = res_ref, 2 ** -7 * res_ref.abs() + 1e-6
    else:
        ref = addend.float() + res_ref.bfloat16().float()
        tol = 2 ** -7 * (addend.float().abs() + 2 * res_ref.abs()) + 1e-6
    assert ((out.cpu().float() - ref).abs() <= tol).all()


def test_decode_graph_matches_eager():
    """DecodeGraph replays decode_next exactly, across MLA and local layers,
    and keeps the state consistent with eager steps in between."""
    from parrot import ModelConfig, Parrot
    from parrot.decode_graph import DecodeGraph
    _say("decode graph vs eager")
    torch.manual_seed(3)
    model = Parrot(ModelConfig(n_layers=4, moe_backend="grouped_hip", depth_backend="hip",
                               collect_router_stats=False)).to(device="cuda",
                                                               dtype=torch.bfloat16).eval()
    prompt = torch.randint(0, 32768, (2, 40), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.inference_mode():
        logits, state = model.prefill(prompt)
        eager_state = copy.deepcopy(state)
        nxt = logits[:, -1].argmax(-1, keepdim=True)
        graph = DecodeGraph(model, state)
        assert state.position == 40 and int(state.position_device.item()) == 40
        a, e = nxt.clone(), nxt.clone()
        for step in range(5):
            a = graph.step(a).clone()
            e, eager_state = model.decode_next(e, eager_state)
            assert torch.equal(a, e), step
        # an eager step on the graph's state, then replays continue in step
        a, state = model.decode_next(a, state)
        e, eager_state = model.decode_next(e, eager_state)
        for step in range(2):
            a = graph.step(a).clone()
            e, eager_state = model.decode_next(e, eager_state)
            assert torch.equal(a, e), step
        assert state.position == eager_state.position == 48
        assert int(state.position_device.item()) == 48
        for mine, theirs in zip(state.layers, eager_state.layers):
            for name in ("key", "value", "latent"):
                if hasattr(mine, name):
                    assert torch.equal(getattr(mine, name)[:, :48] if name == "latent" else
                                       getattr(mine, name)[:, :, :48],
                                       getattr(theirs, name)[:, :48] if name == "latent" else
                                       getattr(theirs, name)[:, :, :48])


def test_decode_graph_feeds_tokens_back_in_place():
    """Greedy generation feeds each step's output back: the tokens land in
    the graph's input buffer (no copy before the next replay), and the steps
    still equal eager decoding."""
    from parrot import ModelConfig, Parrot
    from parrot.decode_graph import DecodeGraph
    _say("decode graph in-place token feedback")
    torch.manual_seed(5)
    model = Parrot(ModelConfig(n_layers=4, moe_backend="grouped_hip", depth_backend="hip",
                               collect_router_stats=False)).to(device="cuda",
                                                               dtype=torch.bfloat16).eval()
    prompt = torch.randint(0, 32768, (1, 24), generator=torch.Generator().manual_seed(5)).cuda()
    with torch.inference_mode():
        logits, state = model.prefill(prompt)
        eager_state = copy.deepcopy(state)
        e = logits[:, -1].argmax(-1, keepdim=True)
        graph = DecodeGraph(model, state)
        a = graph.step(e.clone())
        assert a.data_ptr() == graph.ids.data_ptr() and a.shape == (1, 1)
        e, eager_state = model.decode_next(e, eager_state)
        assert torch.equal(a, e)
        for step in range(4):
            a = graph.step(a)
            e, eager_state = model.decode_next(e, eager_state)
            assert torch.equal(a, e), step
        assert int(state.position_device.item()) == eager_state.position == 29


@pytest.mark.parametrize("tokens,k,n,with_addend", [(1, 768, 768, True), (3, 768, 768, False),
                                                    (16, 1024, 16, True), (8, 128, 2048, True)])
def test_decode_linear(tokens, k, n, with_addend):
    """The decode GEMV + addend against fp32 CPU products of the same bf16
    operands: one bf16 rounding of an fp32 sum (order aside), then the bf16
    addend sum."""
    from parrot import hip_moe
    _say(f"decode linear T={tokens} k={k} n={n} addend={with_addend}")
    g = torch.Generator().manual_seed(700 + tokens + n)
    x = torch.randn(tokens, 1, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * k ** -0.5).bfloat16()
    addend = torch.randn(tokens, 1, n, generator=g).bfloat16() if with_addend else None
    with torch.no_grad():
        out = hip_moe.decode_linear(x.cuda(), w.cuda(), None if addend is None else addend.cuda())
    assert out.shape == (tokens, 1, n) and out.dtype == torch.bfloat16
    res = x.float() @ w.float().T
    if addend is None:
        ref, tol = res, 2 ** -7 * res.abs() + 1e-6
    else:
        ref = addend.float() + res.bfloat16().float()
        tol = 2 ** -7 * (addend.float().abs() + 2 * res.abs()) + 1e-6
    assert ((out.cpu().float() - ref).abs() <= tol).all()


@pytest.mark.parametrize("tokens,sources", [(1, 2), (5, 9), (16, 4)])
def test_mla_decode_in_mixes_its_input(tokens, sources):
    """The MLA decode projections from a depth mix equal depth_mix_norm
    followed by the x path, bit for bit."""
    from test_gpu_moe import _Depth, _Norm
    from parrot import hip_moe
    dim, width, r = 768, 1024, 128
    _say(f"mla decode in with its input mix T={tokens} S={sources}")
    g = torch.Generator().manual_seed(500 + tokens)
    wq = (torch.randn(width, dim, generator=g) * 0.05).bfloat16().cuda()
    wkv = (torch.randn(r, dim, generator=g) * 0.05).bfloat16().cuda()
    torch.manual_seed(600 + sources)
    depth = _Depth(dim).cuda().bfloat16()
    norm = _Norm(dim).cuda().bfloat16()
    src = [(torch.randn(tokens, 1, dim, generator=g) * (1 + s)).bfloat16().cuda()
           for s in range(sources)]
    with torch.no_grad():
        h = hip_moe.depth_mix_norm(depth, [s.view(tokens, dim) for s in src], norm)
        q_ref, lat_ref = hip_moe.mla_decode_in(h.view(tokens, 1, dim), wq, wkv)
        q, lat = hip_moe.mla_decode_in(None, wq, wkv, mix=(depth, src, norm))
    assert torch.equal(q, q_ref) and torch.equal(lat, lat_ref)


@pytest.mark.parametrize("tokens,sources,position", [(1, 3, 0), (4, 9, 150), (16, 1, 299)])
def test_decode_qkv(tokens, sources, position):
    """The decode q|k|v projection + RoPE: from x, against the fused MFMA
    projection + RoPE (the fp32 sums differ in order, so the bf16 values may
    differ in the last place); from a depth mix, equal bit for bit to
    depth_mix_norm followed by the x path."""
    from test_gpu_moe import _Depth, _Norm
    from test_gpu_proj import _packed
    from parrot import hip_moe
    from parrot.model import ModelConfig, _rope_tables
    cfg = ModelConfig()
    H, Hk, d, dim = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.dim
    n = (H + 2 * Hk) * d
    _say(f"decode qkv T={tokens} S={sources} p={position}")
    g = torch.Generator().manual_seed(200 + tokens)
    w = (torch.randn(n, dim, generator=g) * dim ** -0.5).bfloat16().cuda()
    x = torch.randn(tokens, 1, dim, generator=g).bfloat16().cuda()
    cos, sin = _rope_tables(cfg, torch.empty(0, device="cuda"))
    pos = torch.tensor([position], dtype=torch.int32, device="cuda")
    torch.manual_seed(300 + sources)
    depth = _Depth(dim).cuda().bfloat16()
    norm = _Norm(dim).cuda().bfloat16()
    src = [(torch.randn(tokens, 1, dim, generator=g) * (1 + s)).bfloat16().cuda()
           for s in range(sources)]
    with torch.no_grad():
        q, k, v = hip_moe.decode_qkv(x, w, cos, sin, H, Hk, d, pos)
        q2, k2, v2 = hip_moe.proj_rope_qkv(x, _packed(w), cos, sin, H, Hk, d, start_device=pos)
        h = hip_moe.depth_mix_norm(depth, [s.view(tokens, dim) for s in src], norm)
        qh, kh, vh = hip_moe.decode_qkv(h.view(tokens, 1, dim), w, cos, sin, H, Hk, d, pos)
        qm, km, vm = hip_moe.decode_qkv(None, w, cos, sin, H, Hk, d, pos, mix=(depth, src, norm))
    assert q.shape == q2.shape and k.shape == k2.shape and v.shape == v2.shape
    for got, ref in ((q, q2), (k, k2), (v, v2)):
        assert (got.float() - ref.float()).abs().max() <= 2 ** -6 * ref.float().abs().max()
    assert torch.equal(qm, qh) and torch.equal(km, kh) and torch.equal(vm, vh)


@pytest.mark.parametrize("tokens,position", [(1, 0), (5, 150), (16, 299)])
def test_decode_qkv_embeds_its_input(tokens, position):
    """The first layer's q|k|v launch that gathers its input rows from the
    token ids: the rows it stores equal the embedding lookup, and q / k / v
    equal the one-source mix path over those rows, bit for bit.  Ids outside
    the table read the nearest row (the first and last tokens here)."""
    from test_gpu_moe import _Depth, _Norm
    from parrot import hip_moe
    from parrot.model import ModelConfig, _rope_tables
    cfg = ModelConfig()
    H, Hk, d, dim, vocab = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.dim, 1000
    n = (H + 2 * Hk) * d
    _say(f"decode qkv with its embedding T={tokens} p={position}")
    g = torch.Generator().manual_seed(400 + tokens)
    w = (torch.randn(n, dim, generator=g) * dim ** -0.5).bfloat16().cuda()
    table = torch.randn(vocab, dim, generator=g).bfloat16().cuda()
    ids = torch.randint(0, vocab, (tokens, 1), generator=g)
    ids[0, 0] = vocab - 1
    rows = table[ids.view(-1)].view(tokens, 1, dim)
    if tokens > 1:
        ids[-1, 0] = vocab + 7  # nearest row: vocab - 1
        rows[-1, 0] = table[vocab - 1]
    ids = ids.cuda()
    cos, sin = _rope_tables(cfg, torch.empty(0, device="cuda"))
    pos = torch.tensor([position], dtype=torch.int32, device="cuda")
    torch.manual_seed(500 + tokens)
    depth = _Depth(dim).cuda().bfloat16()
    norm = _Norm(dim).cuda().bfloat16()
    out = torch.full((tokens, 1, dim), float("nan"), dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        qe, ke, ve = hip_moe.decode_qkv(None, w, cos, sin, H, Hk, d, pos,
                                        mix=(depth, [out], norm), embed=(ids, table))
        qm, km, vm = hip_moe.decode_qkv(None, w, cos, sin, H, Hk, d, pos,
                                        mix=(depth, [rows], norm))
    assert torch.equal(out, rows)
    assert torch.equal(qe, qm) and torch.equal(ke, km) and torch.equal(ve, vm)


@pytest.mark.parametrize("tokens,sources,with_addend", [
    (1, 1, True), (1, 4, False), (3, 9, True), (8, 5, True), (16, 9, False)])
def test_decode_moe_mixes_its_input(tokens, sources, with_addend):
    """The decode MoE that makes its input rows itself (depth mix + norm of
    the sources, per token inside the launch) equals depth_mix_norm followed
    by the decode MoE, bit for bit: the same arithmetic in the same order."""
    from moe_cases import inputs, moe_module
    from test_gpu_moe import _Depth, _Norm
    from parrot import hip_moe
    _say(f"decode moe with its input mix T={tokens} S={sources} addend={with_addend}")
    torch.manual_seed(60 + tokens + sources)
    module = moe_module(16, seed=13)
    depth = _Depth(768).cuda().bfloat16()
    norm = _Norm(768).cuda().bfloat16()
    src = [inputs(tokens, seed=70 + s) * (1 + s) for s in range(sources)]
    addend = inputs(tokens, seed=90) if with_addend else None
    with torch.no_grad():
        h = hip_moe.depth_mix_norm(depth, src, norm)
        ref, ref_idx, ref_w = hip_moe.decode_experts(module, h, addend=addend)
        out, idx, w = hip_moe.decode_experts(module, None, addend=addend,
                                             mix=(depth, src, norm))
    assert torch.equal(idx, ref_idx) and torch.equal(w, ref_w)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("tokens,experts,skewed,with_addend", [
    (1, 16, False, False), (2, 16, False, True), (5, 32, True, False), (8, 16, False, True),
    (16, 3, False, True), (16, 32, False, False)])
def test_decode_moe_fused(tokens, experts, skewed, with_addend):
    """The two-launch decode MoE against the fp32 oracle (parrot/model.py:
    520-551) on its own routing, and its routing against the oracle's top-2
    of fp32 logits."""
    import numpy as np
    from moe_cases import MAX_ABS, MEAN_ABS, error_stats, inputs, moe_module, oracle_moe, skew_bias
    from parrot import hip_moe
    _say(f"decode moe T={tokens} E={experts} skew={skewed} addend={with_addend}")
    module = moe_module(experts, seed=11)
    x = inputs(tokens, seed=11 + tokens)
    bias = skew_bias(experts) if skewed else None
    addend = inputs(tokens, seed=12) if with_addend else None
    with torch.no_grad():
        out, idx, w = hip_moe.decode_experts(module, x, addend=addend, logit_bias=bias)
        delta, idx2, w2 = hip_moe.decode_experts(module, x, logit_bias=bias)
    assert torch.equal(idx, idx2) and torch.equal(w, w2)
    if with_addend:  # the same two roundings as `addend + delta`
        assert torch.equal(out, addend + delta)
    idx_np = idx.cpu().numpy()
    ref_routed, ref_idx, ref_w, logits = oracle_moe(
        module, x, logit_bias=None if bias is None else bias.numpy())
    # routing: identical wherever the fp32 logits leave a visible margin
    biased = logits.numpy() + (0 if bias is None else bias.numpy())
    top = np.sort(biased, axis=-1)[:, ::-1]
    clear = (top[:, 0] - top[:, 1] > 1e-4) & (top[:, 1] - top[:, 2] > 1e-4) if experts > 2 else \
        np.ones(tokens, bool)
    assert (idx_np[clear] == ref_idx[clear]).all()
    np.testing.assert_allclose(w.cpu().numpy()[clear], ref_w[clear], atol=2e-6)
    ref, _, _, _ = oracle_moe(module, x, indices=idx_np, weights=w.cpu().numpy())
    mx, mean = error_stats(delta, ref)
    _say(f"  max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx <= MAX_ABS and mean <= MEAN_ABS


@pytest.mark.parametrize("rows,vocab,dim", [(1, 32768, 768), (3, 32768, 768), (16, 32768, 768),
                                            (5, 1000, 64), (2, 777, 2048)])
def test_vocab_argmax(rows, vocab, dim):
    """Greedy tokens from fp32 logits equal the fp32 argmax wherever the top
    two logits are not within fp32 reassociation of each other, and exact
    ties go to the lower index."""
    from parrot import hip_moe
    _say(f"vocab argmax rows={rows} vocab={vocab} dim={dim}")
    g = torch.Generator().manual_seed(rows * 7 + dim)
    w = (torch.randn(vocab, dim, generator=g) * 0.02).bfloat16()
    h = torch.randn(rows, dim, generator=g).bfloat16()
    # planted exact tie: rows 11 and 900 % vocab of the head are identical
    # and made the best match of h[0]
    w[11] = h[0] * 0.05
    w[(900 % (vocab - 12)) + 12] = w[11]
    with torch.no_grad():
        got = hip_moe.vocab_argmax(h.cuda(), w.cuda()).cpu()
    logits = h.double() @ w.double().T
    top2 = logits.topk(2, dim=-1)
    ref = logits.argmax(-1)
    assert got[0].item() == 11
    clear = (top2.values[:, 0] - top2.values[:, 1]) > 1e-4
    assert torch.equal(got[clear], ref[clear])


def test_vocab_argmax_advances_the_position():
    """The argmax launch increments the device position counter once (the
    decode step's last launch advances it) and picks the same tokens."""
    from parrot import hip_moe
    gen = torch.Generator().manual_seed(11)
    h = torch.randn(3, 768, generator=gen).bfloat16().cuda()
    w = (torch.randn(32768, 768, generator=gen) * 0.02).bfloat16().cuda()
    pos = torch.full((1,), 41, dtype=torch.int32, device="cuda")
    with torch.no_grad():
        plain = hip_moe.vocab_argmax(h, w)
        with_advance = hip_moe.vocab_argmax(h, w, advance=pos)
    assert torch.equal(plain, with_advance)
    assert int(pos.item()) == 42


@pytest.mark.parametrize("dim,experts", [(2048, 32), (64, 3)])
def test_decode_moe_router_weights_in_memory_or_lds(dim, experts):
    """dim 2048 at E = 32 (128 KB of router weights, read from memory) and
    dim 64 at E = 3 (staged in LDS, a partial 1 KB group): the decode MoE
    against the fp32 oracle on its own routing."""
    from moe_cases import MAX_ABS, MEAN_ABS, error_stats, inputs, moe_module, oracle_moe
    from parrot import hip_moe
    _say(f"decode moe dim={dim} E={experts}")
    module = moe_module(experts, seed=13, dim=dim)
    x = inputs(3, seed=13, dim=dim)
    with torch.no_grad():
        out, idx, w = hip_moe.decode_experts(module, x)
        full = hip_moe.route(module, x, collect_stats=False)
    ref, _, _, _ = oracle_moe(module, x, indices=idx.cpu().numpy(), weights=w.cpu().numpy())
    mx, mean = error_stats(out, ref)
    assert mx <= MAX_ABS and mean <= MEAN_ABS
    assert torch.equal(full.indices, idx)


def test_decode_with_32_heads_runs_undeferred(monkeypatch):
    """A model with 32 query heads (more lanes than the pending decode mix
    takes) decodes on the undeferred path: the per-head kernel is never
    called, and prefill + decode steps match the fp32 oracle forced to the
    HIP top-2 choices (the full-model rule of tests/parity.py)."""
    from oracle import parrot_fp32
    from parity import RouteRecorder, format_report, logits_report
    from parrot import ModelConfig, Parrot, hip_moe
    _say("decode with 32 query heads (undeferred)")

    def refuse(*a, **k):
        raise AssertionError("the deferred per-head decode attention was chosen")
    monkeypatch.setattr(hip_moe, "decode_attention_heads", refuse)
    torch.manual_seed(7)
    cfg = ModelConfig(n_layers=4, n_heads=32, n_kv_heads=4, head_dim=64,
                      moe_backend="grouped_hip", depth_backend="hip", collect_router_stats=False)
    model = Parrot(cfg).to(device="cuda", dtype=torch.bfloat16).eval()
    prompt = torch.randint(0, 32768, (1, 24), generator=torch.Generator().manual_seed(7))
    rec = RouteRecorder(monkeypatch)
    logits, state = model.prefill(prompt.cuda())
    got, tokens = [logits.float().cpu()], []
    for _ in range(4):
        tokens.append(got[-1][:, -1].argmax(-1, keepdim=True))
        logits, state = model.decode_step(tokens[-1].cuda(), state)
        got.append(logits.float().cpu())
    hip_idx = rec.stop()
    forced = parrot_fp32.ParrotFP32(cfg, model.state_dict(), forced_routing=hip_idx)
    ref, f_state = forced.prefill(prompt)
    refs = [ref]
    for tok in tokens:
        refs.append(forced.decode_step(tok, f_state))
    r = logits_report(torch.cat([g.reshape(-1, g.shape[-1]) for g in got]),
                      torch.cat([x.reshape(-1, x.shape[-1]) for x in refs]), 0.03)
    _say(f"  vs forced oracle: {format_report(r)}")
    assert r["clear_miss"] == 0 and r["max_abs"] <= 0.03 and r["mean_abs"] <= 3.5e-3


def test_vocab_argmax_is_batch_invariant():
    """A row's greedy token does not depend on the batch it is decoded in:
    rows with planted near-ties (two head rows whose logits differ by one
    bf16 ulp of one weight, within fp32 reassociation of each other) give
    the same token alone and inside batches of 2, 5 and 16 rows."""
    from parrot import hip_moe
    _say("vocab argmax batch invariance")
    g = torch.Generator().manual_seed(13)
    vocab, dim, n = 32768, 768, 32
    w = (torch.randn(vocab, dim, generator=g) * 0.02).bfloat16()
    h = torch.randn(n, dim, generator=g).bfloat16()
    for i in range(n):
        a, b = 100 + 2 * i, 101 + 2 * i
        w[a] = (h[i].float() * 0.05).bfloat16()
        w[b] = w[a]
        j = int(h[i].float().abs().argmin())  # the smallest |h| element: a tiny logit change
        w[b, j] = (w[a, j:j + 1].view(torch.int16) + 1).view(torch.bfloat16)[0]  # one bf16 ulp
    wc, hc = w.cuda(), h.cuda()
    with torch.no_grad():
        alone = torch.stack([hip_moe.vocab_argmax(hc[i:i + 1], wc)[0] for i in range(n)]).cpu()
        for size in (2, 5, 16):
            for start in range(0, n - size + 1, size):
                batch = hip_moe.vocab_argmax(hc[start:start + size], wc).cpu()
                assert torch.equal(batch, alone[start:start + size]), (size, start)
    assert all(int(alone[i]) in (100 + 2 * i, 101 + 2 * i) for i in range(n))


def test_eager_decode_step_rejects_out_of_range_ids():
    """Eager decode_step raises on a token id outside the embedding table, as
    the reference's nn.Embedding does, instead of reading a clamped row (the
    fused first-layer launch clamps, for graph replay)."""
    from parrot import ModelConfig, Parrot
    torch.manual_seed(3)
    model = Parrot(ModelConfig(n_layers=4, moe_backend="grouped_hip", depth_backend="hip",
                               collect_router_stats=False)).to(device="cuda",
                                                               dtype=torch.bfloat16).eval()
    prompt = torch.randint(0, 32768, (2, 8), generator=torch.Generator().manual_seed(3)).cuda()
    _, state = model.prefill(prompt)
    for bad in (32768, -1):
        ids = torch.tensor([[5], [bad]], device="cuda")
        with pytest.raises(IndexError):
            model.decode_step(ids, state)
    assert state.position == 8
    logits, state = model.decode_step(torch.tensor([[5], [7]], device="cuda"), state)
    assert state.position == 9 and torch.isfinite(logits.float()).all()
    # The forward and prefill gather their rows in the first launch, which
    # clamps too: eager calls raise before it.
    for bad in (32768, -1):
        ids = prompt.clone()
        ids[1, 3] = bad
        with torch.no_grad(), pytest.raises(IndexError):
            model(ids)
        with pytest.raises(IndexError):
            model.prefill(ids)
