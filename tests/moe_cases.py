"""Shared builders for MoE-layer parity cases (the BASELINE configurations).

C2: 256 tokens, E=32, near-uniform routing (seed 1).
C3: 4096 tokens, E=32, logit bias +4.0 on expert 0 and +2.0 on expert 1.
C4: 512 tokens, E=16 (the full model's layer shape).
C5: 1..8 tokens, E=16 (decode).
Weights ~ N(0, 0.02), activations ~ N(0, 1), as BASELINE.json states.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import layers

DIM, HIDDEN, SHARED = 768, 512, 256
MAX_ABS, MEAN_ABS = 2e-2, 2e-3  # bf16 MoE output vs fp32


def moe_module(experts: int, seed: int, dim=DIM, hidden=HIDDEN, shared=SHARED,
               device="cuda", dtype=torch.bfloat16):
    from parrot.model import ModelConfig, MoE
    cfg = ModelConfig(dim=dim, expert_dim=hidden, shared_expert_dim=shared, n_experts=experts,
                      moe_backend="grouped_hip", depth_backend="hip",
                      collect_router_stats=False)
    gen = torch.Generator().manual_seed(seed)
    module = MoE(cfg)
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    return module.to(device=device, dtype=dtype).eval()


def inputs(tokens: int, seed: int, dim=DIM, device="cuda", dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed + 1000)
    return torch.randn(tokens, dim, generator=gen).to(device=device, dtype=dtype)


def skew_bias(experts: int) -> torch.Tensor:
    bias = torch.zeros(experts)
    bias[0], bias[1] = 4.0, 2.0
    return bias


def oracle_moe(module, x: torch.Tensor, indices=None, weights=None, logit_bias=None):
    """fp32 oracle on the module's (bf16) weights upcast."""
    cpu = {k: v.detach().float().cpu() for k, v in module.state_dict().items()}
    experts = [(cpu[f"experts.{e}.gate.weight"], cpu[f"experts.{e}.up.weight"],
                cpu[f"experts.{e}.down.weight"]) for e in range(module.cfg.n_experts)]
    shared = (cpu["shared.gate.weight"], cpu["shared.up.weight"], cpu["shared.down.weight"])
    return layers.moe_layer(x.float().cpu(), cpu["router.weight"], experts, shared,
                            None if logit_bias is None else np.asarray(logit_bias),
                            indices, weights)


def error_stats(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    d = (got.float().cpu() - ref.float().cpu()).abs()
    return float(d.max()), float(d.mean())
