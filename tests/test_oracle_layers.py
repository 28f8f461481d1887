"""Pin the fp32 layer oracle with closed forms and invariants.

RMSNorm (parrot/model.py:125-127), depth mix (:149-155), SwiGLU (:443-448)
and the MoE layer (:520-551) each meet a check that a dropped term, a wrong
sign or a transposed operand would fail.
"""
import math

import numpy as np
import torch

from oracle import layers, routing


def test_rms_norm_closed_form():
    x = torch.full((3, 16), 2.0)
    w = torch.arange(16, dtype=torch.float32)
    y = layers.rms_norm(x, w, 1e-6)
    np.testing.assert_allclose(y.numpy(), (2.0 / math.sqrt(4.0 + 1e-6)) * w.expand(3, 16).numpy(),
                               rtol=1e-6)
    # scale invariance: rms_norm(a x) == rms_norm(x) for a > 0 (eps -> 0)
    r = torch.randn(5, 64)
    np.testing.assert_allclose(layers.rms_norm(7 * r, torch.ones(64), 1e-12).numpy(),
                               layers.rms_norm(r, torch.ones(64), 1e-12).numpy(), atol=1e-5)


def test_depth_mix_invariants():
    torch.manual_seed(0)
    src = [torch.randn(4, 32) for _ in range(5)]
    w = torch.rand(32) + 0.5
    # one source -> identity
    np.testing.assert_allclose(layers.depth_mix(src[:1], torch.randn(32), w, 1e-6).numpy(),
                               src[0].numpy(), atol=1e-6)
    # zero query -> uniform average
    np.testing.assert_allclose(layers.depth_mix(src, torch.zeros(32), w, 1e-6).numpy(),
                               torch.stack(src).mean(0).numpy(), atol=1e-6)
    # a query strongly aligned with source 2's normalised key picks source 2
    key = layers.rms_norm(src[2], w, 1e-6)[0]
    q = 200.0 * key / key.norm()
    out = layers.depth_mix([s[:1] for s in src], q, w, 1e-6)
    np.testing.assert_allclose(out.numpy(), src[2][:1].numpy(), atol=1e-4)
    # brute force per token
    q = torch.randn(32)
    out = layers.depth_mix(src, q, w, 1e-6)
    for t in range(4):
        scores = []
        for s in src:
            v = s[t]
            scores.append(float(((v / torch.sqrt((v * v).mean() + 1e-6)) * w * q).sum()))
        a = np.exp(np.array(scores) - max(scores))
        a /= a.sum()
        ref = sum(float(a[i]) * src[i][t] for i in range(5))
        np.testing.assert_allclose(out[t].numpy(), ref.numpy(), atol=1e-5)


def test_swiglu_scalar_form():
    torch.manual_seed(1)
    x = torch.randn(3, 8)
    g, u, d = torch.randn(4, 8), torch.randn(4, 8), torch.randn(8, 4)
    out = layers.swiglu(x, g, u, d)
    for t in range(3):
        h = []
        for j in range(4):
            a = float(x[t] @ g[j])
            b = float(x[t] @ u[j])
            h.append(a / (1 + math.exp(-a)) * b)
        ref = [sum(d[m, j].item() * h[j] for j in range(4)) for m in range(8)]
        np.testing.assert_allclose(out[t].numpy(), ref, rtol=1e-5, atol=1e-6)


def test_moe_layer_token_major_bruteforce():
    """Expert-loop form (index_add over torch.where rows) equals a per-token sum."""
    torch.manual_seed(2)
    dim, hidden, hs, experts, tokens = 16, 8, 4, 6, 20
    x = torch.randn(tokens, dim)
    router = torch.randn(experts, dim)
    ex = [(torch.randn(hidden, dim), torch.randn(hidden, dim), torch.randn(dim, hidden))
          for _ in range(experts)]
    sh = (torch.randn(hs, dim), torch.randn(hs, dim), torch.randn(dim, hs))
    out, idx, w, logits = layers.moe_layer(x, router, ex, sh)
    np.testing.assert_allclose(logits.numpy(), (x @ router.T).numpy(), rtol=1e-5, atol=1e-5)
    for t in range(tokens):
        ref = layers.swiglu(x[t:t + 1], *sh)[0]
        for k in range(2):
            ref = ref + float(w[t, k]) * layers.swiglu(x[t:t + 1], *ex[idx[t, k]])[0]
        np.testing.assert_allclose(out[t].numpy(), ref.numpy(), rtol=1e-5, atol=1e-5)
    i2, w2, _ = routing.top2(logits.numpy())
    np.testing.assert_array_equal(idx, i2)
