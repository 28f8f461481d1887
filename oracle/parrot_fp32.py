"""TEST INFRASTRUCTURE ONLY: functional fp32 restatement of the Parrot model.

Runs the reference's ``moe_backend="pytorch"`` semantics on CPU in fp32 over
a state_dict (reference jkpdino/parrot-h200-worker parrot/model.py):
  embedding + Block AttnRes residual stream           :667-710
  sliding-window RoPE GQA attention                   :167-328
  MLA attention (decode: explicit latent expansion,   :331-432
    mathematically equal to the absorbed form)
  MoE with shared expert                              :463-569
  tied vocabulary head                                :714-715
  prefill / decode_step with KV and latent caches    :748-931
Attention is written out as softmax(q k^T / sqrt(d) + mask) v with explicit
band / causal masks, independent of scaled_dot_product_attention.
"""
from __future__ import annotations

import math

import numpy as np
import torch
from torch.nn import functional as F

from . import layers, routing


class ParrotFP32:
    """``forced_routing``: optional list of int64 [tokens, 2] top-2 index
    arrays, consumed one per MoE call in execution order; a MoE layer then
    uses those experts (weights renormalised over its own fp32 softmax at
    those indices, as the reference's top-2 weights are, model.py:525-527)
    instead of its own top-2.  Feeding the indices another implementation
    chose separates the discontinuity of top-2 selection at near-tied router
    logits from the arithmetic precision of everything else."""

    def __init__(self, cfg, state_dict: dict[str, torch.Tensor], forced_routing=None):
        self.c = cfg
        self.p = {k: v.detach().float().cpu() for k, v in state_dict.items()}
        self.forced_routing = None if forced_routing is None else list(forced_routing)

    # ---- building blocks ------------------------------------------------------

    def _w(self, name: str) -> torch.Tensor:
        return self.p[name]

    def _rope(self, x: torch.Tensor, start: int) -> torch.Tensor:
        c = self.c
        t = x.shape[-2]
        inv = c.rope_theta ** (-torch.arange(0, c.head_dim, 2).float() / c.head_dim)
        ang = torch.arange(start, start + t).float()[:, None] * inv
        cos, sin = ang.cos(), ang.sin()
        even, odd = x[..., 0::2], x[..., 1::2]
        out = torch.empty_like(x)
        out[..., 0::2] = even * cos - odd * sin
        out[..., 1::2] = even * sin + odd * cos
        return out

    @staticmethod
    def _attend(q, k, v, allowed: torch.Tensor, scale: float) -> torch.Tensor:
        """q [b, H, tq, d]; k, v [b, Hk, tk, d] shared by H / Hk query heads."""
        rep = q.shape[1] // k.shape[1]
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        scores = (q @ k.transpose(-1, -2)) * scale
        scores = scores.masked_fill(~allowed, float("-inf"))
        return scores.softmax(-1) @ v

    def _local_prefill(self, i: int, h: torch.Tensor):
        c, pre = self.c, f"blocks.{i}.attention."
        b, t, _ = h.shape
        q = F.linear(h, self._w(pre + "q.weight")).view(b, t, c.n_heads, c.head_dim).transpose(1, 2)
        k = F.linear(h, self._w(pre + "k.weight")).view(b, t, c.n_kv_heads, c.head_dim).transpose(1, 2)
        v = F.linear(h, self._w(pre + "v.weight")).view(b, t, c.n_kv_heads, c.head_dim).transpose(1, 2)
        q, k = self._rope(q, 0), self._rope(k, 0)
        qi = torch.arange(t)[:, None]
        ki = torch.arange(t)[None, :]
        allowed = (ki <= qi) & (ki > qi - c.window_size)
        y = self._attend(q, k, v, allowed, 1.0 / math.sqrt(c.head_dim))
        out = F.linear(y.transpose(1, 2).reshape(b, t, -1), self._w(pre + "out.weight"))
        return out, k, v

    def _mla_prefill(self, i: int, h: torch.Tensor):
        c, pre = self.c, f"blocks.{i}.attention."
        b, t, _ = h.shape

        def heads(y):
            return y.view(b, t, c.n_heads, c.head_dim).transpose(1, 2)

        latent = F.linear(h, self._w(pre + "kv_down.weight"))
        q = heads(F.linear(h, self._w(pre + "q.weight")))
        k = heads(F.linear(latent, self._w(pre + "k_up.weight")))
        v = heads(F.linear(latent, self._w(pre + "v_up.weight")))
        allowed = torch.arange(t)[None, :] <= torch.arange(t)[:, None]
        y = self._attend(q, k, v, allowed, 1.0 / math.sqrt(c.head_dim))
        return F.linear(y.transpose(1, 2).reshape(b, t, -1), self._w(pre + "out.weight")), latent

    def moe(self, i: int, h: torch.Tensor, logit_bias=None):
        pre = f"blocks.{i}.moe."
        experts = [(self._w(f"{pre}experts.{e}.gate.weight"), self._w(f"{pre}experts.{e}.up.weight"),
                    self._w(f"{pre}experts.{e}.down.weight")) for e in range(self.c.n_experts)]
        shared = (self._w(pre + "shared.gate.weight"), self._w(pre + "shared.up.weight"),
                  self._w(pre + "shared.down.weight"))
        indices = weights = None
        if self.forced_routing is not None:
            indices = np.ascontiguousarray(self.forced_routing.pop(0), dtype=np.int64).reshape(-1, 2)
            logits = layers.router_logits(h.reshape(-1, h.shape[-1]), self._w(pre + "router.weight"))
            bias = None if logit_bias is None else np.asarray(logit_bias, dtype=np.float32)
            _, _, probs = routing.top2(logits.numpy(), bias, want_probs=True)
            p = np.take_along_axis(probs, indices, axis=1)
            weights = p / (p[:, :1] + p[:, 1:])
        out, idx, w, logits = layers.moe_layer(h, self._w(pre + "router.weight"), experts, shared,
                                               logit_bias, indices, weights)
        return out.view_as(h), idx, w, logits

    def _norm(self, name: str, x):
        return layers.rms_norm(x, self._w(name + ".weight"), self.c.norm_eps)

    def _mix(self, j: int, sources):
        return layers.depth_mix(sources, self._w(f"depth_mix.{j}.query"),
                                self._w(f"depth_mix.{j}.norm.weight"), self.c.norm_eps)

    def _is_global(self, i: int) -> bool:
        return (i + 1) % self.c.global_every == 0

    # ---- full passes ----------------------------------------------------------

    def _run(self, x: torch.Tensor, attention, capture: dict | None = None):
        """Residual stream over all blocks; ``attention(i, h)`` returns the
        attention delta of block i."""
        c = self.c
        attnres = c.residual == "attnres"
        completed, partial = [x], None
        index = 0
        for i in range(c.n_layers):
            for is_moe in (False, True):
                if attnres:
                    sources = completed + ([] if partial is None else [partial])
                    pre = self._mix(index, sources)
                    if capture is not None:
                        capture.setdefault("depth", []).append(pre)
                else:
                    pre = x
                if is_moe:
                    h = self._norm(f"blocks.{i}.moe_norm", pre)
                    delta, idx, w, logits = self.moe(i, h)
                    if capture is not None:
                        capture.setdefault("moe_in", []).append(h)
                        capture.setdefault("moe_out", []).append(delta)
                        capture.setdefault("indices", []).append(idx)
                        capture.setdefault("logits", []).append(logits)
                else:
                    delta = attention(i, self._norm(f"blocks.{i}.attention_norm", pre))
                if attnres:
                    partial = delta if partial is None else partial + delta
                    if (index + 1) % c.depth_block_size == 0:
                        completed.append(partial)
                        partial = None
                else:
                    x = x + delta
                index += 1
        if attnres:
            x = self._mix(index, completed + ([] if partial is None else [partial]))
            if capture is not None:
                capture.setdefault("depth", []).append(x)
        return x

    def head(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(self._norm("final_norm", x), self._w("embedding.weight"))

    def forward(self, ids: torch.Tensor, capture: dict | None = None) -> torch.Tensor:
        x = self._w("embedding.weight")[ids]

        def attention(i, h):
            return (self._mla_prefill(i, h)[0] if self._is_global(i)
                    else self._local_prefill(i, h)[0])

        return self.head(self._run(x, attention, capture))

    def prefill(self, ids: torch.Tensor, capture: dict | None = None):
        """(logits of the last position [b, 1, V], cache state)."""
        c = self.c
        b, t = ids.shape
        state = {"position": t, "layers": []}

        def attention(i, h):
            if self._is_global(i):
                out, latent = self._mla_prefill(i, h)
                cache = torch.zeros(b, c.max_seq_len, c.kv_latent_dim)
                cache[:, :t] = latent
                state["layers"].append(("mla", cache))
            else:
                out, k, v = self._local_prefill(i, h)
                kc = torch.zeros(b, c.n_kv_heads, c.max_seq_len, c.head_dim)
                vc = torch.zeros_like(kc)
                kc[:, :, :t] = k
                vc[:, :, :t] = v
                state["layers"].append(("local", kc, vc))
            return out

        x = self._run(self._w("embedding.weight")[ids], attention, capture)
        return self.head(x[:, -1:]), state

    def decode_step(self, ids: torch.Tensor, state: dict,
                    capture: dict | None = None) -> torch.Tensor:
        """Logits [b, 1, V] for one new token per sequence; updates state."""
        c = self.c
        b = ids.shape[0]
        p = state["position"]

        def attention(i, h):
            pre = f"blocks.{i}.attention."
            layer = state["layers"][i]
            if layer[0] == "local":
                _, kc, vc = layer
                q = F.linear(h, self._w(pre + "q.weight")).view(b, 1, c.n_heads, c.head_dim).transpose(1, 2)
                k = F.linear(h, self._w(pre + "k.weight")).view(b, 1, c.n_kv_heads, c.head_dim).transpose(1, 2)
                v = F.linear(h, self._w(pre + "v.weight")).view(b, 1, c.n_kv_heads, c.head_dim).transpose(1, 2)
                q, k = self._rope(q, p), self._rope(k, p)
                kc[:, :, p:p + 1] = k
                vc[:, :, p:p + 1] = v
                lo = max(0, p - c.window_size + 1)
                allowed = torch.ones(1, p + 1 - lo, dtype=torch.bool)
                y = self._attend(q, kc[:, :, lo:p + 1], vc[:, :, lo:p + 1], allowed,
                                 1.0 / math.sqrt(c.head_dim))
            else:
                _, lc = layer
                lc[:, p:p + 1] = F.linear(h, self._w(pre + "kv_down.weight"))
                latent = lc[:, :p + 1]
                k = F.linear(latent, self._w(pre + "k_up.weight")).view(b, p + 1, c.n_heads, c.head_dim).transpose(1, 2)
                v = F.linear(latent, self._w(pre + "v_up.weight")).view(b, p + 1, c.n_heads, c.head_dim).transpose(1, 2)
                q = F.linear(h, self._w(pre + "q.weight")).view(b, 1, c.n_heads, c.head_dim).transpose(1, 2)
                allowed = torch.ones(1, p + 1, dtype=torch.bool)
                y = self._attend(q, k, v, allowed, 1.0 / math.sqrt(c.head_dim))
            return F.linear(y.transpose(1, 2).reshape(b, 1, -1), self._w(pre + "out.weight"))

        x = self._run(self._w("embedding.weight")[ids], attention, capture)
        state["position"] = p + 1
        return self.head(x)


def tiny_config():
    """The build's definition of the reference README's ``--tiny`` config."""
    from types import SimpleNamespace
    return SimpleNamespace(
        vocab_size=32768, dim=64, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=16,
        kv_latent_dim=32, global_every=4, window_size=32, max_seq_len=128,
        n_experts=8, top_k=2, expert_dim=128, shared_expert_dim=64, residual="attnres",
        depth_block_size=4, rope_theta=10000.0, norm_eps=1e-6, local_query_chunk=16)


def logit_agreement(a: np.ndarray, b: np.ndarray) -> float:
    """Fraction of positions whose argmax agrees."""
    return float((a.reshape(-1, a.shape[-1]).argmax(-1) == b.reshape(-1, b.shape[-1]).argmax(-1)).mean())
