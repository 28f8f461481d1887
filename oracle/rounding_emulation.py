"""TEST INFRASTRUCTURE ONLY: the fp32 oracle with the HIP forward's bf16
rounding points switched on one by one (CPU), to attribute the full-model
argmax disagreement between a bf16 forward and the fp32 reference.

Rounding points of the HIP forward (each a toggle below):
  act      every activation a kernel writes in bf16: the depth-mix output and
           its RMSNorm, q / k / v (before and after RoPE), the attention
           output, every projection output, the expert hidden rows
           (parrot/kernels/moe_bf16.metal:675), the shared expert's output
           and each route-weighted expert output (the rows the down
           projection writes; parrot/metal_moe.py:407-409 rounds expert
           outputs to bf16, parrot/model.py:550 each weighted contribution),
           and the MoE output;
  stream   the AttnRes partial sums (partial + delta rounded to bf16);
  head_in  the final RMSNorm output fed to the vocabulary head;
  logit    the vocabulary head's output.
Routing is the oracle's own fp32 top-2 of the (rounded) MoE input, or forced
to given indices (``force``).  Everything else follows oracle/parrot_fp32.py
(reference jkpdino/parrot-h200-worker parrot/model.py:658-746).

``acc64`` accumulates every linear map in float64 before its fp32 result is
rounded: the same rounding points with another accumulation order.  Two such
bf16 forwards differ only where a pre-rounding value sits within fp32
reassociation of a bf16 rounding boundary; comparing them measures how far
that alone carries a bf16 forward (its noise floor).
"""
from __future__ import annotations

import math

import numpy as np
import torch
from torch.nn import functional as F

from . import routing


def bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


def _same(x: torch.Tensor) -> torch.Tensor:
    return x


def _linear(acc64: bool):
    if not acc64:
        return F.linear
    return lambda x, w: F.linear(x.double(), w.double()).float()


def forward(o, ids: torch.Tensor, *, act=True, stream=True, head_in=True, logit=True,
            force=None, capture: list | None = None, acc64: bool = False) -> torch.Tensor:
    """Logits of ParrotFP32 ``o`` on ``ids`` with the selected rounding
    points; ``capture`` collects each MoE layer's top-2 indices."""
    lin = _linear(acc64)
    ra = bf16 if act else _same
    rs = bf16 if stream else _same
    c = o.c
    x = o._w("embedding.weight")[ids]
    completed, partial = [x], None
    index = 0
    for i in range(c.n_layers):
        for is_moe in (False, True):
            sources = completed + ([] if partial is None else [partial])
            pre = ra(o._mix(index, sources))
            if is_moe:
                h = ra(o._norm(f"blocks.{i}.moe_norm", pre))
                delta = _moe(o, i, h, ra, None if force is None else force[i], capture, lin)
            else:
                h = ra(o._norm(f"blocks.{i}.attention_norm", pre))
                delta = _attention(o, i, h, ra, lin)
            partial = delta if partial is None else rs(partial + delta)
            if (index + 1) % c.depth_block_size == 0:
                completed.append(partial)
                partial = None
            index += 1
    mixed = ra(o._mix(index, completed + ([] if partial is None else [partial])))
    h = o._norm("final_norm", mixed)
    h = bf16(h) if head_in else h
    out = lin(h, o._w("embedding.weight"))
    return bf16(out) if logit else out


def _moe(o, i, h, ra, forced, capture, lin=F.linear):
    pre = f"blocks.{i}.moe."
    flat = h.reshape(-1, h.shape[-1])
    logits = lin(flat, o._w(pre + "router.weight"))
    if forced is None:
        idx, w, _ = routing.top2(logits.numpy())
    else:
        idx = np.ascontiguousarray(forced, dtype=np.int64)
        _, _, probs = routing.top2(logits.numpy(), want_probs=True)
        p = np.take_along_axis(probs, idx, axis=1)
        w = p / (p[:, :1] + p[:, 1:])
    if capture is not None:
        capture.append(idx)

    def swiglu(rows, name):
        hidden = ra(F.silu(lin(rows, o._w(name + "gate.weight"))) *
                    lin(rows, o._w(name + "up.weight")))
        return lin(hidden, o._w(name + "down.weight"))

    out = ra(swiglu(flat, pre + "shared."))
    it = torch.from_numpy(idx)
    wt = torch.from_numpy(np.asarray(w, dtype=np.float32))
    for e in range(o.c.n_experts):
        rows, slots = torch.where(it == e)
        if rows.numel():
            out = out.index_add(0, rows, ra(swiglu(flat[rows], f"{pre}experts.{e}.") *
                                           wt[rows, slots, None]))
    return ra(out).view_as(h)


def _attention(o, i, h, ra, lin=F.linear):
    c, pre = o.c, f"blocks.{i}.attention."
    b, t, _ = h.shape

    def heads(y, n):
        return y.view(b, t, n, c.head_dim).transpose(1, 2)

    if (i + 1) % c.global_every:
        q = heads(ra(lin(h, o._w(pre + "q.weight"))), c.n_heads)
        k = heads(ra(lin(h, o._w(pre + "k.weight"))), c.n_kv_heads)
        v = heads(ra(lin(h, o._w(pre + "v.weight"))), c.n_kv_heads)
        q, k = ra(o._rope(q, 0)), ra(o._rope(k, 0))
        qi, ki = torch.arange(t)[:, None], torch.arange(t)[None, :]
        allowed = (ki <= qi) & (ki > qi - c.window_size)
    else:
        latent = ra(lin(h, o._w(pre + "kv_down.weight")))
        q = heads(ra(lin(h, o._w(pre + "q.weight"))), c.n_heads)
        k = heads(ra(lin(latent, o._w(pre + "k_up.weight"))), c.n_heads)
        v = heads(ra(lin(latent, o._w(pre + "v_up.weight"))), c.n_heads)
        allowed = torch.arange(t)[None, :] <= torch.arange(t)[:, None]
    y = ra(o._attend(q, k, v, allowed, 1.0 / math.sqrt(c.head_dim)))
    return ra(lin(y.transpose(1, 2).reshape(b, t, -1), o._w(pre + "out.weight")))
