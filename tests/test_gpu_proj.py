"""GPU parity of the dense projection kernels (the attention layers' linear
maps, parrot/model.py:167-230 and 331-432 in the reference).

y = x W^T is checked against an fp32 CPU product of the same bf16 operands
(one bf16 rounding of the output plus fp32 reassociation), with hipBLASLt's
bf16 F.linear as a control.  The residual-add, transposed and RoPE epilogues
must reproduce, bit for bit, the plain projection followed by the separate
operation they replace: bf16(addend + bf16(y)) (the rounding of the
reference's attention_output_decode_bf16, parrot/kernels/moe_bf16.metal:
1364-1389), a transpose, and the stand-alone RoPE kernel.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _operands(rows, k, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * k ** -0.5).bfloat16()
    return x, w


class _Owner(torch.nn.Module):
    """Holds the packed-weight cache for one test weight."""


def _packed(w):
    from parrot import hip_moe
    return hip_moe.pack_linear(_Owner().eval(), "_w", (w.cuda(),))


@pytest.mark.parametrize("rows,k,n", [(512, 768, 1152), (512, 768, 768), (512, 768, 128),
                                      (512, 128, 768), (1, 768, 1152), (17, 768, 768),
                                      (1000, 2048, 64), (300, 1024, 2048), (33, 64, 16)])
def test_proj_matches_fp32(rows, k, n):
    from parrot import hip_moe
    _say(f"proj rows={rows} k={k} n={n}")
    x, w = _operands(rows, k, n, rows + k + n)
    with torch.no_grad():
        got = hip_moe.proj(x.cuda(), _packed(w), n).float().cpu()
        control = torch.nn.functional.linear(x.cuda(), w.cuda()).float().cpu()
    ref = x.float() @ w.float().T
    bound = x.float().abs() @ w.float().abs().T
    tol = 2 ** -8 * ref.abs() + 1e-6 * k * bound + 1e-6
    err = (got - ref).abs()
    _say(f"  max-abs {err.max():.3e} mean-abs {err.mean():.3e}; control max-abs "
         f"{(control - ref).abs().max():.3e}")
    assert (err <= tol).all()


def test_proj_strided_input_and_addend():
    """A row-strided input is read in place; the addend epilogue equals the
    separate bf16 add exactly, also written over the addend itself."""
    from parrot import hip_moe
    _say("proj strided input + addend")
    x, w = _operands(300, 768, 768, 7)
    wide = torch.zeros(300, 1024, dtype=torch.bfloat16)
    wide[:, 128:896] = x
    a = torch.randn(300, 768, generator=torch.Generator().manual_seed(8)).bfloat16()
    packed = _packed(w)
    with torch.no_grad():
        xs = wide.cuda()[:, 128:896]
        plain = hip_moe.proj(x.cuda(), packed, 768)
        strided = hip_moe.proj(xs, packed, 768)
        added = hip_moe.proj(x.cuda(), packed, 768, addend=a.cuda())
    assert torch.equal(plain, strided)
    assert torch.equal(added.cpu(), (a.float() + plain.float().cpu()).bfloat16())


@pytest.mark.parametrize("batch,seq", [(2, 512), (3, 13), (1, 1), (2, 100)])
def test_proj_transposed(batch, seq):
    from parrot import hip_moe
    _say(f"proj transposed b={batch} t={seq}")
    x, w = _operands(batch * seq, 128, 768, seq)
    packed = _packed(w)
    keys = hip_moe.padded_keys(seq)
    with torch.no_grad():
        plain = hip_moe.proj(x.cuda(), packed, 768).view(batch, seq, 768)
        vt = hip_moe.proj_transposed(x.cuda().view(batch, seq, 128), packed, 768, keys)
    assert vt.shape == (batch, 768, keys)
    assert torch.equal(vt[..., :seq], plain.transpose(1, 2))


@pytest.mark.parametrize("batch,seq,start,device_start,vt", [
    (1, 512, 0, None, True), (2, 37, 5, None, False), (3, 1, 0, 41, False),
    (2, 64, 0, 100, True), (1, 16, 3, None, True)])
def test_proj_rope_qkv(batch, seq, start, device_start, vt):
    """Fused projection + RoPE == projection, then the RoPE kernel."""
    from parrot import hip_moe
    from parrot.model import ModelConfig, _rope_tables
    cfg = ModelConfig()
    H, Hk, d = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    n = (H + 2 * Hk) * d
    _say(f"proj rope qkv b={batch} t={seq} start={start} device={device_start} vt={vt}")
    x, w = _operands(batch * seq, cfg.dim, n, seq + start)
    packed = _packed(w)
    cos, sin = _rope_tables(cfg, torch.empty(0, device="cuda"))
    pos = None if device_start is None else torch.tensor([device_start], dtype=torch.int32,
                                                         device="cuda")
    keys = hip_moe.padded_keys(seq) if vt else 0
    xc = x.cuda().view(batch, seq, cfg.dim)
    with torch.no_grad():
        q, k, v = hip_moe.proj_rope_qkv(xc, packed, cos, sin, H, Hk, d, start, pos, keys)
        qkv = hip_moe.proj(xc, packed, n)
        q2, k2, v2 = hip_moe.rope_qkv(qkv, cos, sin, H, Hk, d, start, False, pos, keys)
    assert torch.equal(q, q2) and torch.equal(k, k2)
    assert torch.equal(v[..., :seq] if vt else v, v2[..., :seq] if vt else v2)


def _valid_fragments(b, h, t, d):
    """Masks of the key positions a fragment-order K / V holds for t keys."""
    from parrot import hip_moe
    ones = torch.ones(b, h, t, d, dtype=torch.bfloat16, device="cuda")
    km, vm = hip_moe.pack_kv_fragments(ones, ones)
    return km != 0, vm != 0


@pytest.mark.parametrize("batch,seq", [(1, 512), (2, 37), (3, 1), (1, 96)])
def test_proj_rope_qkv_fragments(batch, seq):
    """The fragment outputs hold exactly the row-major q|k|v path's k and v."""
    from parrot import hip_moe
    from parrot.model import ModelConfig, _rope_tables
    cfg = ModelConfig()
    H, Hk, d = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    n = (H + 2 * Hk) * d
    _say(f"proj rope qkv fragments b={batch} t={seq}")
    x, w = _operands(batch * seq, cfg.dim, n, 5 * seq)
    packed = _packed(w)
    cos, sin = _rope_tables(cfg, torch.empty(0, device="cuda"))
    xc = x.cuda().view(batch, seq, cfg.dim)
    with torch.no_grad():
        q, kf, vf, k, v = hip_moe.proj_rope_qkv_frag(xc, packed, cos, sin, H, Hk, d)
        q1, kf1, vf1, k1, v1 = hip_moe.proj_rope_qkv_frag(xc, packed, cos, sin, H, Hk, d,
                                                          cache_kv=False)
        q2, k2, v2 = hip_moe.proj_rope_qkv(xc, packed, cos, sin, H, Hk, d)
    assert k1 is None and v1 is None
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    assert torch.equal(q1, q2)
    kr, vr = hip_moe.pack_kv_fragments(k2, v2)
    km, vm = _valid_fragments(batch, Hk, seq, d)
    assert torch.equal(kf[km], kr[km]) and torch.equal(vf[vm], vr[vm])
    assert torch.equal(kf1[km], kr[km]) and torch.equal(vf1[vm], vr[vm])


@pytest.mark.parametrize("batch,seq,values", [(1, 512, False), (1, 512, True), (2, 45, True),
                                              (2, 45, False), (1, 3, True)])
def test_proj_fragments(batch, seq, values):
    """The MLA up-projections stored as fragment-order K / V."""
    from parrot import hip_moe
    _say(f"proj fragments b={batch} t={seq} values={values}")
    heads, d, r = 8, 96, 128
    x, w = _operands(batch * seq, r, heads * d, seq + int(values))
    packed = _packed(w)
    xc = x.cuda().view(batch, seq, r)
    with torch.no_grad():
        got = hip_moe.proj_frag(xc, packed, heads * d, d, values)
        plain = hip_moe.proj(xc, packed, heads * d).view(batch, seq, heads, d).transpose(1, 2)
    ref = hip_moe.pack_kv_fragments(plain, plain)[1 if values else 0]
    mask = _valid_fragments(batch, heads, seq, d)[1 if values else 0]
    assert torch.equal(got[mask], ref[mask])


@pytest.mark.parametrize("batch,seq", [(1, 512), (2, 45), (1, 3)])
def test_proj_kv_fragments(batch, seq):
    """[Wk; Wv] in one launch from a row-strided latent == two single launches."""
    from parrot import hip_moe
    _say(f"proj kv fragments b={batch} t={seq}")
    heads, d, r = 8, 96, 128
    x, w = _operands(batch * seq, r, 2 * heads * d, seq + 11)
    wide = torch.zeros(batch * seq, 896, dtype=torch.bfloat16)
    wide[:, 768:] = x
    latent = wide.cuda().view(batch, seq, 896)[..., 768:]
    with torch.no_grad():
        kf, vf = hip_moe.proj_kv_frag(latent, _packed(w), heads * d, d)
        k1 = hip_moe.proj_frag(x.cuda().view(batch, seq, r), _packed(w[:heads * d]), heads * d,
                               d, False)
        v1 = hip_moe.proj_frag(x.cuda().view(batch, seq, r), _packed(w[heads * d:]), heads * d,
                               d, True)
    km, vm = _valid_fragments(batch, heads, seq, d)
    assert torch.equal(kf[km], k1[km]) and torch.equal(vf[vm], v1[vm])
