"""Full-model parity rules shared by the GPU model tests.

A bf16 forward differs from the fp32 oracle in two ways:
  * arithmetic precision: every activation is rounded to bf16, so logits move
    by ~1e-2 at most;
  * top-2 routing: where two router logits of a token are nearly tied, the
    bf16 and fp32 inputs can select different experts.  That changes the
    token's MoE output by a whole expert's contribution, and through
    attention the later positions too.  It is the divergence class the
    routing contract names (given identical logits the top-2 is bit-exact).

So every full-model check runs the oracle twice: free (its own fp32 top-2),
and forced to the top-2 choices the HIP path made (``RouteRecorder``).
  * Against the forced oracle the logits must be within tight bounds.  Every
    HIP choice must equal the forced oracle's fp32 top-2, except at router
    near-ties.
  * Against the free oracle the greedy argmax must agree on every position
    whose fp32 top-1/top-2 gap exceeds a margin.  The margin is taken above
    the largest gap error measured with free routing.  A raw agreement floor
    must also hold.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import routing


class RouteRecorder:
    """Records the top-2 indices of every HIP MoE layer in execution order,
    whichever entry computed them (route, route_top2, the routing depth mix,
    or the fused decode MoE)."""

    def __init__(self, monkeypatch):
        from parrot import hip_moe
        self.indices: list[np.ndarray] = []
        self.active = True
        route, top2, mix_route, decode = (hip_moe.route, hip_moe.route_top2,
                                          hip_moe.depth_mix_norm_route, hip_moe.decode_experts)

        def rec(ix):
            if self.active:  # copying to the host synchronises: never under capture
                self.indices.append(ix.detach().cpu().numpy().reshape(-1, 2).copy())

        def route_rec(*a, **k):
            r = route(*a, **k)
            rec(r.indices)
            return r

        def top2_rec(*a, **k):
            r = top2(*a, **k)
            rec(r.indices)
            return r

        def mix_route_rec(*a, **k):
            h, r = mix_route(*a, **k)
            rec(r.indices)
            return h, r

        def decode_rec(*a, **k):
            out = decode(*a, **k)
            rec(out[1])
            return out

        monkeypatch.setattr(hip_moe, "route", route_rec)
        monkeypatch.setattr(hip_moe, "route_top2", top2_rec)
        monkeypatch.setattr(hip_moe, "depth_mix_norm_route", mix_route_rec)
        monkeypatch.setattr(hip_moe, "decode_experts", decode_rec)

    def take(self) -> list[np.ndarray]:
        out, self.indices = self.indices, []
        return out

    def stop(self) -> list[np.ndarray]:
        """Stop recording (before a graph capture) and return the records."""
        self.active = False
        return self.take()


def say(msg: str) -> None:
    print(msg, flush=True)


def logits_report(got: torch.Tensor, ref: torch.Tensor, margin: float) -> dict:
    """Argmax agreement (raw and on positions whose fp32 top-1/top-2 gap
    exceeds ``margin``), logits max/mean abs error, and the error of the
    top-1/top-2 gap (how far the HIP logits move the fp32 decision)."""
    got = got.float().cpu().reshape(-1, got.shape[-1])
    ref = ref.float().cpu().reshape(-1, ref.shape[-1])
    top = ref.topk(2, dim=-1)
    gap = top.values[:, 0] - top.values[:, 1]
    agree = got.argmax(-1) == top.indices[:, 0]
    got_gap = got.gather(1, top.indices[:, :1])[:, 0] - got.gather(1, top.indices[:, 1:])[:, 0]
    gap_err = (got_gap - gap).abs()
    clear = gap > margin
    d = (got - ref).abs()
    return dict(agree=agree.float().mean().item(), n=agree.numel(),
                clear_agree=agree[clear].float().mean().item() if clear.any() else 1.0,
                clear_n=int(clear.sum()), clear_miss=int((~agree[clear]).sum()),
                max_abs=d.max().item(), mean_abs=d.mean().item(),
                gap_err_max=gap_err.max().item(), gap_err_q99=gap_err.quantile(0.99).item())


def format_report(r: dict) -> str:
    return (f"argmax {r['agree']:.4f} of {r['n']}, on clear gaps {r['clear_agree']:.4f} "
            f"of {r['clear_n']} ({r['clear_miss']} missed); logits max-abs {r['max_abs']:.3e} "
            f"mean-abs {r['mean_abs']:.3e}; gap error max {r['gap_err_max']:.4f} "
            f"q99 {r['gap_err_q99']:.4f}")


def routing_report(hip: list[np.ndarray], logits: list[torch.Tensor]) -> dict:
    """Compares each HIP top-2 choice with the fp32 top-2 of the forced
    oracle's router logits on the same layer.

    A differing expert set is allowed only where the fp32 2nd and 3rd logits
    are near-tied; a swapped order only where the 1st and 2nd are.  Reports
    the number of differing tokens and the largest fp32 margin at such a
    difference."""
    flips = swaps = total = 0
    worst = 0.0
    for idx, lg in zip(hip, logits):
        lg = lg.float().cpu().numpy().reshape(idx.shape[0], -1)
        ref_idx, _, _ = routing.top2(lg)
        srt = np.sort(lg, axis=-1)[:, ::-1]
        set_diff = np.sort(idx, -1) != np.sort(ref_idx, -1)
        set_diff = set_diff.any(-1)
        order_diff = (idx != ref_idx).any(-1) & ~set_diff
        if set_diff.any():
            worst = max(worst, float((srt[set_diff, 1] - srt[set_diff, 2]).max()))
        if order_diff.any():
            worst = max(worst, float((srt[order_diff, 0] - srt[order_diff, 1]).max()))
        flips += int(set_diff.sum())
        swaps += int(order_diff.sum())
        total += idx.shape[0]
    return dict(flips=flips, swaps=swaps, tokens=total, worst_margin=worst)
