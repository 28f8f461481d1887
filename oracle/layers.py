"""TEST INFRASTRUCTURE ONLY: fp32 CPU restatements of the hot-path layers.

Every function computes in fp32 on whatever values it is given (bf16
tensors are upcast, so only the arithmetic precision differs from the HIP
kernels).  Reference formulas (jkpdino/parrot-h200-worker):
  rms_norm   parrot/model.py:125-127
  depth_mix  parrot/model.py:149-155 (keys RMS-normalised, values raw)
  swiglu     parrot/model.py:443-448
  moe_layer  parrot/model.py:520-527 (router + top-2) and 545-551
             (shared expert first, then every expert's rows in
             torch.where order, index_add of weighted outputs)
"""
from __future__ import annotations

import numpy as np
import torch
from torch.nn import functional as F

from . import routing


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    y = x.float()
    y = y * torch.rsqrt(y.square().mean(-1, keepdim=True) + eps)
    return y * weight.float()


def depth_mix(sources: list[torch.Tensor], query: torch.Tensor, norm_weight: torch.Tensor,
              eps: float) -> torch.Tensor:
    values = torch.stack([s.float() for s in sources], dim=0)
    keys = rms_norm(values, norm_weight, eps)
    scores = (keys * query.float()).sum(-1)
    alpha = scores.softmax(dim=0)
    return (alpha.unsqueeze(-1) * values).sum(0)


def swiglu(x: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
           down: torch.Tensor) -> torch.Tensor:
    x = x.float()
    return F.linear(F.silu(F.linear(x, gate.float())) * F.linear(x, up.float()), down.float())


def router_logits(x: torch.Tensor, router: torch.Tensor) -> torch.Tensor:
    return F.linear(x.float(), router.float())


def moe_layer(x: torch.Tensor, router: torch.Tensor, experts, shared, logit_bias=None,
              indices: np.ndarray | None = None, weights: np.ndarray | None = None):
    """fp32 MoE layer.  experts: list of (gate, up, down); shared: (gate, up, down).

    Routing comes from the C oracle on fp32 logits (+ logit_bias), unless
    ``indices``/``weights`` are given.  Returns (out [T, dim] fp32,
    indices int64 [T, 2], weights fp32 [T, 2], logits fp32 [T, E])."""
    flat = x.reshape(-1, x.shape[-1]).float()
    logits = router_logits(flat, router)
    if indices is None:
        bias = None if logit_bias is None else np.asarray(logit_bias, dtype=np.float32)
        indices, weights, _ = routing.top2(logits.numpy(), bias)
    idx = torch.from_numpy(np.asarray(indices, dtype=np.int64))
    w = torch.from_numpy(np.asarray(weights, dtype=np.float32))
    result = swiglu(flat, *shared)
    for e, (g, u, d) in enumerate(experts):
        rows, slots = torch.where(idx == e)
        if rows.numel():
            result = result.index_add(0, rows, swiglu(flat[rows], g, u, d) * w[rows, slots, None])
    return result, np.asarray(indices), np.asarray(weights), logits
