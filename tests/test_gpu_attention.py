"""GPU parity of the causal / sliding-window attention kernel against an
fp32 CPU restatement of scaled_dot_product_attention with the reference's
masks (parrot/model.py:264-295 band mask, 350-360 causal), with PyTorch's
own bf16 flash attention on the GPU as a control for the error bf16
operands allow."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _reference(q, k, v, scale, window):
    b, H, t, d = q.shape
    rep = H // k.shape[1]
    k = k.float().repeat_interleave(rep, dim=1)
    v = v.float().repeat_interleave(rep, dim=1)
    i = torch.arange(t)[:, None]
    j = torch.arange(t)[None, :]
    mask = (j <= i) & (j > i - window)
    s = (q.float() @ k.transpose(-1, -2)) * scale
    s = s.masked_fill(~mask, float("-inf"))
    return (torch.softmax(s, dim=-1) @ v).transpose(1, 2).reshape(b, t, H * d)


@pytest.mark.parametrize("b,H,Hk,t,d,window,strided", [
    (1, 8, 2, 512, 96, 2048, False),   # local layer of the bs1x512 forward
    (2, 8, 8, 77, 96, 4096, True),     # MLA layer: heads view of [b, t, H*d]
    (1, 4, 1, 300, 64, 100, False),    # band narrower than the sequence
    (2, 2, 2, 33, 128, 33, False),
    (3, 8, 2, 1, 96, 2048, False),
    (1, 8, 2, 17, 96, 5, True),
])
def test_causal_attention(b, H, Hk, t, d, window, strided):
    from parrot import hip_moe
    _say(f"attention b={b} H={H} Hk={Hk} t={t} d={d} window={window} strided={strided}")
    g = torch.Generator().manual_seed(t * 31 + d)
    if strided:
        q = torch.randn(b, t, H * d, generator=g).bfloat16().view(b, t, H, d).transpose(1, 2)
        k = torch.randn(b, t, Hk * d, generator=g).bfloat16().view(b, t, Hk, d).transpose(1, 2)
        v = torch.randn(b, t, Hk * d, generator=g).bfloat16().view(b, t, Hk, d).transpose(1, 2)
    else:
        q = torch.randn(b, H, t, d, generator=g).bfloat16()
        k = torch.randn(b, Hk, t, d, generator=g).bfloat16()
        v = torch.randn(b, Hk, t, d, generator=g).bfloat16()
    scale = d ** -0.5
    with torch.no_grad():
        got = hip_moe.causal_attention(q.cuda(), k.cuda(), v.cuda(), scale=scale,
                                       window=window).float().cpu()
        # the same through transposed values whose padding holds non-finite bytes
        vt = torch.full((b, Hk, d, hip_moe.padded_keys(t) + 8), float("nan"),
                        dtype=torch.bfloat16, device="cuda")
        vt[..., :t] = v.cuda().transpose(-1, -2)
        got_t = hip_moe.causal_attention(q.cuda(), k.cuda(), vt=vt, scale=scale,
                                         window=window).float().cpu()
    assert torch.equal(got, got_t)
    ref = _reference(q, k, v, scale, window)
    err = (got - ref).abs()
    _say(f"  max-abs {err.max():.3e} mean-abs {err.mean():.3e}")
    assert err.max() <= 1e-2 and err.mean() <= 1e-3
    if window >= t:  # PyTorch's bf16 attention as the control
        rep = H // Hk
        with torch.no_grad():
            ctl = F.scaled_dot_product_attention(
                q.cuda(), k.cuda().repeat_interleave(rep, 1).contiguous(),
                v.cuda().repeat_interleave(rep, 1).contiguous(), is_causal=True)
        ctl = ctl.float().cpu().transpose(1, 2).reshape(b, t, H * d)
        ctl_err = (ctl - ref).abs()
        _say(f"  control max-abs {ctl_err.max():.3e} mean-abs {ctl_err.mean():.3e}")
        assert err.mean() <= 2 * ctl_err.mean() + 1e-5


def _padded_nan(x, t):
    """[b, h, t, d] -> [b, h, ceil(t / 32) * 32, d] with non-finite padding keys."""
    from parrot import hip_moe
    b, h, _, d = x.shape
    out = torch.full((b, h, hip_moe.key_blocks(t) * 32, d), float("nan"), dtype=x.dtype)
    out[:, :, :t] = x
    return out


@pytest.mark.parametrize("b,H,Hk,t,d,window", [
    (1, 8, 2, 512, 96, 2048), (2, 8, 8, 77, 96, 4096), (1, 4, 1, 300, 64, 100),
    (2, 2, 2, 33, 128, 33), (3, 8, 2, 1, 96, 2048), (1, 8, 2, 1000, 96, 256)])
def test_causal_attention_fragments(b, H, Hk, t, d, window):
    """K and V in fragment order (padding keys non-finite) give exactly the
    strided kernel's output; the torch packer and the kernel agree on the
    layout because the results match."""
    from parrot import hip_moe
    _say(f"attention fragments b={b} H={H} Hk={Hk} t={t} d={d} window={window}")
    g = torch.Generator().manual_seed(t * 7 + d)
    q = torch.randn(b, H, t, d, generator=g).bfloat16()
    k = torch.randn(b, Hk, t, d, generator=g).bfloat16()
    v = torch.randn(b, Hk, t, d, generator=g).bfloat16()
    kf, vf = hip_moe.pack_kv_fragments(_padded_nan(k, t).cuda(), _padded_nan(v, t).cuda())
    with torch.no_grad():
        strided = hip_moe.causal_attention(q.cuda(), k.cuda(), v.cuda(), scale=d ** -0.5,
                                           window=window)
        frag = hip_moe.causal_attention_frag(q.cuda(), kf, vf, kv_heads=Hk, scale=d ** -0.5,
                                             window=window)
    assert torch.equal(frag, strided)
    if t >= 300:
        ref = _reference(q, k, v, d ** -0.5, window)
        err = (frag.float().cpu() - ref).abs()
        _say(f"  max-abs {err.max():.3e} mean-abs {err.mean():.3e}")
        assert err.max() <= 1e-2 and err.mean() <= 1e-3


@pytest.mark.parametrize("b,H,Hk,t,d,dim,window", [
    (1, 8, 2, 512, 96, 768, 2048),   # local layer of the bs1x512 forward
    (1, 8, 8, 512, 96, 768, 4096),   # MLA layer (one kv head per head)
    (2, 8, 2, 77, 64, 512, 40),      # ragged rows, band narrower than the sequence
    (1, 8, 4, 33, 128, 1024, 33),
    (3, 8, 2, 1, 96, 768, 2048),
])
def test_causal_attention_out_heads(b, H, Hk, t, d, dim, window):
    """The attention kernel with the output projection deferred per head:
    contributions[.., h, :] equal float64 products of the attention output
    (the same kernel's bf16 y) with the head's columns of the output weight
    within fp32 accumulation error; bf16 of their sum is the projection."""
    from parrot import hip_moe
    _say(f"attention out heads b={b} H={H} Hk={Hk} t={t} d={d} dim={dim} window={window}")
    g = torch.Generator().manual_seed(t * 3 + d + dim)
    q = torch.randn(b, H, t, d, generator=g).bfloat16()
    k = torch.randn(b, Hk, t, d, generator=g).bfloat16()
    v = torch.randn(b, Hk, t, d, generator=g).bfloat16()
    w = (torch.randn(dim, H * d, generator=g) * 0.02).bfloat16()
    kf, vf = hip_moe.pack_kv_fragments(_padded_nan(k, t).cuda(), _padded_nan(v, t).cuda())
    holder = torch.nn.Module()
    holder.out = torch.nn.Linear(H * d, dim, bias=False).cuda().bfloat16()
    with torch.no_grad():
        holder.out.weight.copy_(w)
        packed = hip_moe.pack_linear(holder, "out", (holder.out.weight,))
        y = hip_moe.causal_attention_frag(q.cuda(), kf, vf, kv_heads=Hk, scale=d ** -0.5,
                                          window=window)
        got = hip_moe.causal_attention_frag_out(q.cuda(), kf, vf, packed, dim, kv_heads=Hk,
                                                scale=d ** -0.5, window=window)
        proj = hip_moe.proj(y, packed, dim)
    assert got.shape == (b, t, H, dim) and got.dtype == torch.float32
    yh = y.double().cpu().view(b, t, H, d)
    wh = w.double().view(dim, H, d)
    exact = torch.einsum("bthd,nhd->bthn", yh, wh)
    scale = torch.einsum("bthd,nhd->bthn", yh.abs(), wh.abs())
    err = (got.double().cpu() - exact).abs()
    _say(f"  max err / scale {float((err / scale.clamp_min(1e-30)).max()):.3e}")
    assert bool((err <= 2e-6 * scale + 1e-30).all())
    # bf16(sum over heads) against the one-GEMM projection: the same value
    # up to fp32 reassociation, which moves a rounding boundary now and then
    # (one bf16 ulp of the result, or more where the heads cancel: then by
    # at most fp32 error of the terms' scale)
    summed = got.sum(2).bfloat16().cpu().double()
    ref = proj.cpu().double()
    diff = (summed - ref).abs()
    ulp = torch.maximum(summed.abs(), ref.abs()) * 2 ** -7
    assert bool((diff <= ulp + 1e-5 * scale.sum(2)).all())
    assert float((summed != ref).double().mean()) < 0.02
