"""Parrot XL decoder: PyTorch reference backend plus the MI355X HIP backend.

Public API mirrors the reference package (parrot/__init__.py, parrot/model.py):
``ModelConfig``, ``Parrot`` (``forward``, ``prefill``, ``decode_step``,
``decode_next``, ``parameter_counts``), ``ModelOutput``, ``GenerationState``.

Backends
  * ``moe_backend="pytorch"`` / ``depth_backend="pytorch"``: plain PyTorch on
    any device (training and inference), the semantics of the reference's
    pytorch path (parrot/model.py:109-164, 435-569, 658-931).
  * ``moe_backend="grouped_hip"`` / ``depth_backend="hip"``: the inference
    hot path on MI355X -- router/top-2, deterministic fixed-capacity grouping
    with exact overflow, grouped MFMA SwiGLU experts, combine, RMSNorm and
    Block AttnRes run as HIP kernels (``parrot.hip_moe``).  It takes the place
    of the reference's Apple-Metal ``grouped_mps`` / ``metal`` pair and, like
    it, is inference-only and raises on unsupported inputs instead of falling
    back.

The module tree, parameter names and initialisation order are those of the
reference, so state_dicts are interchangeable and ``torch.manual_seed(s);
Parrot(cfg)`` draws the same weights.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch
from torch import Tensor, nn
from torch.nn import functional as F
from torch.utils.checkpoint import checkpoint

_ROPE_TABLES: dict[tuple, tuple[Tensor, Tensor]] = {}
_WINDOW_MASKS: dict[tuple, list[Tensor]] = {}

MOE_BACKENDS = ("pytorch", "grouped_hip")
DEPTH_BACKENDS = ("pytorch", "hip")
_FOREIGN_BACKENDS = {
    "metal": "Apple-Metal", "dense_mps": "Apple-Metal", "grouped_mps": "Apple-Metal",
    "training_mps": "Apple-Metal training", "training_cuda": "CUDA training",
}


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int = 32768
    dim: int = 768
    n_layers: int = 16
    n_heads: int = 8
    n_kv_heads: int = 2
    head_dim: int = 96
    kv_latent_dim: int = 128
    global_every: int = 4
    window_size: int = 2048  # includes the current position
    max_seq_len: int = 4096
    n_experts: int = 16
    top_k: int = 2
    expert_dim: int = 512
    shared_expert_dim: int = 256
    moe_backend: Literal["pytorch", "grouped_hip"] = "pytorch"
    depth_backend: Literal["pytorch", "hip"] = "pytorch"
    residual: Literal["attnres", "standard"] = "attnres"
    depth_block_size: int = 4  # attention and MoE each count as one module
    rope_theta: float = 10000.0
    norm_eps: float = 1e-6
    aux_loss_weight: float = 0.01
    collect_router_stats: bool = True
    checkpoint_modules: bool = False
    local_query_chunk: int = 256

    @property
    def depth_sources(self) -> int:
        """Sources of the final depth mix: the embedding plus every block sum."""
        modules = 2 * self.n_layers
        return 1 + (modules + self.depth_block_size - 1) // self.depth_block_size

    @property
    def uses_hip(self) -> bool:
        return self.moe_backend == "grouped_hip" or self.depth_backend == "hip"

    def __post_init__(self):
        # Same checks as the reference (parrot/model.py:45-82), with the HIP
        # backend's limits in place of the Metal ones.
        positive = ("vocab_size", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                    "kv_latent_dim", "global_every", "window_size", "max_seq_len",
                    "n_experts", "top_k", "expert_dim", "shared_expert_dim",
                    "depth_block_size", "local_query_chunk")
        for name in positive:
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.n_heads % self.n_kv_heads or self.head_dim % 2:
            raise ValueError("n_heads must divide by n_kv_heads; head_dim must be even")
        if self.top_k > self.n_experts:
            raise ValueError("top_k cannot exceed n_experts")
        if self.residual not in ("attnres", "standard"):
            raise ValueError("residual must be attnres or standard")
        if self.moe_backend in _FOREIGN_BACKENDS:
            raise ValueError(
                f"moe_backend {self.moe_backend!r} is the reference's "
                f"{_FOREIGN_BACKENDS[self.moe_backend]} backend; on MI355X use "
                "'grouped_hip' (inference) or 'pytorch'")
        if self.moe_backend not in MOE_BACKENDS:
            raise ValueError("invalid moe_backend")
        if self.depth_backend == "metal":
            raise ValueError("depth_backend 'metal' is Apple-only; on MI355X use 'hip'")
        if self.depth_backend not in DEPTH_BACKENDS:
            raise ValueError("depth_backend must be pytorch or hip")
        if self.moe_backend == "grouped_hip":
            if self.top_k != 2:
                raise ValueError("grouped_hip requires top_k=2")
            if self.n_experts > 32:
                raise ValueError("grouped_hip supports at most 32 routed experts")
            if any(w % 64 for w in (self.dim, self.expert_dim, self.shared_expert_dim)):
                raise ValueError("grouped_hip requires dim, expert_dim and "
                                 "shared_expert_dim divisible by 64")
        if self.uses_hip and (self.dim % 4 or self.dim > 2048):
            raise ValueError("the HIP norm kernels require dim divisible by four and <= 2048")
        if self.depth_backend == "hip" and self.depth_sources > 9:
            raise ValueError("hip depth mixing supports at most nine sources")
        if self.norm_eps <= 0 or self.rope_theta <= 0 or self.aux_loss_weight < 0:
            raise ValueError("Invalid norm_eps, rope_theta, or aux_loss_weight")


@dataclass
class LocalKVCache:
    key: Tensor    # [batch, kv heads, max positions, head width], RoPE applied
    value: Tensor


@dataclass
class MLALatentCache:
    latent: Tensor  # [batch, max positions, latent width]


@dataclass
class PendingResidual:
    """A decode module output whose final sum is deferred to its consumer
    (reference parrot/model.py:103-106): ``bf16(base + bf16(sum over lanes
    of contributions))``, contributions fp32 [batch, lanes, dim]."""
    base: Tensor | None
    contributions: Tensor


@dataclass
class GenerationState:
    layers: list[LocalKVCache | MLALatentCache]
    position: int
    batch_size: int
    # The same position as a one-element int32 tensor on the cache device,
    # advanced on the device each step; set by prefill on the HIP backend,
    # whose decode kernels read it, so a decode step has static shapes.
    position_device: Tensor | None = None


@dataclass
class ModelOutput:
    logits: Tensor               # [batch, model positions, vocab]
    loss: Tensor | None
    lm_loss: Tensor | None
    aux_loss: Tensor             # unweighted mean over layers
    expert_utilization: Tensor   # [layers, experts], fraction of assignments


def _hip_inference(x: Tensor) -> bool:
    """True where the HIP kernels apply: ROCm bf16 tensors without autograd."""
    return x.device.type == "cuda" and x.dtype == torch.bfloat16 and not torch.is_grad_enabled()


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float, use_hip: bool = False):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps
        self.use_hip = use_hip

    def forward(self, x: Tensor) -> Tensor:
        if self.use_hip and _hip_inference(x):
            from . import hip_moe
            return hip_moe.rms_norm(self, x)
        # fp32 statistics, one rounding back (reference parrot/model.py:125-127)
        y = x.float()
        y = y * torch.rsqrt(y.square().mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class DepthMix(nn.Module):
    """Block AttnRes: attend over earlier block sums with a learned query.

    Keys are RMS-normalised, values are the raw block sums
    (reference parrot/model.py:130-164)."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.query = nn.Parameter(torch.zeros(cfg.dim))
        self.norm = RMSNorm(cfg.dim, cfg.norm_eps, use_hip=cfg.depth_backend == "hip")

    def forward(self, sources: list[Tensor]) -> Tensor:
        if self.cfg.depth_backend == "hip":
            from . import hip_moe
            return hip_moe.depth_mix(self, sources)
        values = torch.stack(sources, dim=0)
        keys = F.rms_norm(values, (self.cfg.dim,), self.norm.weight, self.norm.eps)
        scores = (keys.float() * self.query.float()).sum(-1)
        alpha = scores.softmax(dim=0).to(values.dtype)
        return (alpha.unsqueeze(-1) * values).sum(0)

    def normalized(self, sources: list[Tensor], output_norm: RMSNorm) -> Tensor:
        """``output_norm(self(sources))``; one fused kernel on the HIP backend."""
        if self.cfg.depth_backend == "hip" and _hip_inference(sources[0]):
            from . import hip_moe
            return hip_moe.depth_mix_norm(self, sources, output_norm)
        return output_norm(self(sources))


def _rope_tables(cfg: ModelConfig, like: Tensor) -> tuple[Tensor, Tensor]:
    """cos/sin of position * theta^(-2i/d), computed in fp32 then cast."""
    key = (like.device.type, like.device.index, like.dtype, cfg.max_seq_len, cfg.head_dim,
           cfg.rope_theta)
    tables = _ROPE_TABLES.get(key)
    if tables is None:
        with torch.inference_mode(False):
            inv = cfg.rope_theta ** (
                -torch.arange(0, cfg.head_dim, 2, device=like.device).float() / cfg.head_dim)
            angle = torch.arange(cfg.max_seq_len, device=like.device).float()[:, None] * inv
            tables = (angle.cos().to(like.dtype), angle.sin().to(like.dtype))
        _ROPE_TABLES[key] = tables
    return tables


def _apply_rope(cfg: ModelConfig, x: Tensor, start: int) -> Tensor:
    """Rotate interleaved (even, odd) pairs of the head width."""
    end = start + x.shape[-2]
    if end > cfg.max_seq_len:
        raise ValueError("RoPE position exceeds max_seq_len")
    cos_t, sin_t = _rope_tables(cfg, x)
    cos, sin = cos_t[start:end], sin_t[start:end]
    even, odd = x[..., 0::2], x[..., 1::2]
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), -1).flatten(-2)


def _window_masks(cfg: ModelConfig, t: int, device) -> list[Tensor]:
    """Boolean masks of the query chunks of a sliding-window prefill."""
    key = (device.type, device.index, t, cfg.window_size, cfg.local_query_chunk)
    masks = _WINDOW_MASKS.get(key)
    if masks is None:
        masks = []
        for start in range(0, t, cfg.local_query_chunk):
            end = min(t, start + cfg.local_query_chunk)
            lo = max(0, start - cfg.window_size + 1)
            q = torch.arange(start, end, device=device)[:, None]
            k = torch.arange(lo, end, device=device)[None, :]
            masks.append((k <= q) & (k > q - cfg.window_size))
        _WINDOW_MASKS[key] = masks
    return masks


class LocalGQA(nn.Module):
    """Sliding-window grouped-query attention with RoPE
    (reference parrot/model.py:167-328)."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.q = nn.Linear(cfg.dim, cfg.n_heads * cfg.head_dim, bias=False)
        self.k = nn.Linear(cfg.dim, cfg.n_kv_heads * cfg.head_dim, bias=False)
        self.v = nn.Linear(cfg.dim, cfg.n_kv_heads * cfg.head_dim, bias=False)
        self.out = nn.Linear(cfg.n_heads * cfg.head_dim, cfg.dim, bias=False)

    def _heads(self, y: Tensor, heads: int) -> Tensor:
        b, t, _ = y.shape
        return y.view(b, t, heads, self.cfg.head_dim).transpose(1, 2)

    def _hip(self, x: Tensor) -> bool:
        return self.cfg.uses_hip and _hip_inference(x)

    def _qkv(self, x: Tensor, start: int = 0, expand_kv: bool = False):
        c = self.cfg
        if self._hip(x):
            # One packed projection, then RoPE + head split in one HIP kernel.
            from . import hip_moe
            cos, sin = _rope_tables(c, x.new_empty(0, dtype=torch.float32))
            return hip_moe.rope_qkv(F.linear(x, self._packed_qkv()), cos, sin, c.n_heads,
                                    c.n_kv_heads, c.head_dim, start, expand_kv)
        q = _apply_rope(c, self._heads(self.q(x), c.n_heads), start)
        k = _apply_rope(c, self._heads(self.k(x), c.n_kv_heads), start)
        v = self._heads(self.v(x), c.n_kv_heads)
        return q, k, v

    def fuses_addend(self, x: Tensor) -> bool:
        """True when ``prefill(x, addend)`` folds the residual add into the
        output projection kernel."""
        return self._hip(x) and self._fused_projections()

    def _fused_projections(self) -> bool:
        from . import hip_moe
        c = self.cfg
        width = c.n_heads * c.head_dim
        return (c.head_dim % 4 == 0 and
                hip_moe.proj_supported(c.dim, width + 2 * c.n_kv_heads * c.head_dim) and
                hip_moe.proj_supported(width, c.dim))

    def defers_heads(self, x: Tensor) -> bool:
        """True when ``prefill_heads(x)`` applies: the HIP path with the
        fused projections and a deferrable output projection."""
        from . import hip_moe
        c = self.cfg
        return (self.fuses_addend(x) and
                hip_moe.attention_heads_out_supported(c.n_heads, c.head_dim, c.dim))

    def prefill_heads(self, x: Tensor,
                      need_kv: bool = False) -> tuple[Tensor, Tensor | None, Tensor | None]:
        """The whole-sequence attention output with its projection deferred
        per head: (fp32 contributions [b, t, H, dim], keys, values), the
        contributions' sum over heads, rounded to bf16, being ``prefill(x)[0]``
        up to fp32 summation order (the reference's defer_sum,
        parrot/model.py:301-316); keys and values as ``prefill`` returns them
        when ``need_kv`` (a KV cache is being filled), else None."""
        from . import hip_moe
        c = self.cfg
        cos, sin = _rope_tables(c, x.new_empty(0, dtype=torch.float32))
        q, kf, vf, k, v = hip_moe.proj_rope_qkv_frag(
            x, self._qkv_fragments(), cos, sin, c.n_heads, c.n_kv_heads, c.head_dim,
            cache_kv=need_kv)
        packed = hip_moe.pack_linear(self, "out", (self.out.weight,))
        contributions = hip_moe.causal_attention_frag_out(
            q, kf, vf, packed, c.dim, kv_heads=c.n_kv_heads, scale=c.head_dim ** -0.5,
            window=c.window_size)
        return contributions, k, v

    def _project_out(self, y: Tensor, addend: Tensor | None) -> Tensor:
        """out(y) (+ addend, rounded as bf16(addend + bf16(out(y))))."""
        if self._hip(y) and self._fused_projections():
            from . import hip_moe
            packed = hip_moe.pack_linear(self, "out", (self.out.weight,))
            return hip_moe.proj(y, packed, self.cfg.dim, addend=addend)
        result = self.out(y)
        return result if addend is None else addend + result

    def _qkv_fragments(self) -> Tensor:
        from . import hip_moe
        return hip_moe.pack_linear(self, "qkv", (self.q.weight, self.k.weight, self.v.weight))

    def prefill(self, x: Tensor, addend: Tensor | None = None,
                need_kv: bool = True) -> tuple[Tensor, Tensor | None, Tensor | None]:
        """(out(attention(x)) [+ addend], keys, values) over the whole
        sequence; the HIP path may return None for the keys and values
        unless ``need_kv`` (a KV cache is being filled)."""
        b, t, _ = x.shape
        c = self.cfg
        if self._hip(x):
            from . import hip_moe
            if c.head_dim in hip_moe.ATTENTION_HEAD_DIMS:
                # One HIP kernel for the whole sliding-window causal
                # attention, reading the grouped kv heads in place; the
                # projection (+ RoPE) kernel writes K and V in the attention
                # kernel's fragment order (plus row-major for a cache).
                cos, sin = _rope_tables(c, x.new_empty(0, dtype=torch.float32))
                scale = c.head_dim ** -0.5
                if self._fused_projections():
                    q, kf, vf, k, v = hip_moe.proj_rope_qkv_frag(
                        x, self._qkv_fragments(), cos, sin, c.n_heads, c.n_kv_heads, c.head_dim,
                        cache_kv=need_kv)
                    y = hip_moe.causal_attention_frag(q, kf, vf, kv_heads=c.n_kv_heads,
                                                      scale=scale, window=c.window_size)
                    return self._project_out(y, addend), k, v
                q, k, vt = hip_moe.rope_qkv(F.linear(x, self._packed_qkv()), cos, sin,
                                            c.n_heads, c.n_kv_heads, c.head_dim, 0, False,
                                            vt_keys=hip_moe.padded_keys(t))
                y = hip_moe.causal_attention(q, k, vt=vt, scale=scale, window=c.window_size)
                return self._project_out(y, addend), k, vt[..., :t].transpose(-1, -2)
        result, k, v = self._prefill_torch(x)
        return (result if addend is None else addend + result), k, v

    def _prefill_torch(self, x: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        b, t, _ = x.shape
        c = self.cfg
        if self._hip(x) and t <= c.window_size:
            # Every key of a sequence that fits the window is visible to all
            # later queries, so the banded mask is plain causal: one flash
            # attention call over kv heads expanded by the RoPE kernel.
            q, k, v = self._qkv(x, expand_kv=True)
            y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
            rep = c.n_heads // c.n_kv_heads
            return self.out(y.transpose(1, 2).reshape(b, t, -1)), k[:, ::rep], v[:, ::rep]
        q, k, v = self._qkv(x)
        if t <= c.window_size and t <= c.local_query_chunk:
            y = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        else:
            parts = []
            for mask, start in zip(_window_masks(c, t, x.device),
                                   range(0, t, c.local_query_chunk)):
                end = min(t, start + c.local_query_chunk)
                lo = max(0, start - c.window_size + 1)
                parts.append(F.scaled_dot_product_attention(
                    q[:, :, start:end], k[:, :, lo:end], v[:, :, lo:end],
                    attn_mask=mask, enable_gqa=True))
            y = torch.cat(parts, dim=2)
        return self.out(y.transpose(1, 2).reshape(b, t, -1)), k, v

    def forward(self, x: Tensor, addend: Tensor | None = None) -> Tensor:
        return self.prefill(x, addend, need_kv=False)[0]

    def _packed_qkv(self) -> Tensor:
        cached = self.__dict__.get("_qkv_weight")
        if cached is not None and not torch.is_grad_enabled() and not self.training:
            return cached[1]
        params = (self.q.weight, self.k.weight, self.v.weight)
        version = tuple((p._version, p.device, p.dtype, p.data_ptr()) for p in params)
        if cached is None or cached[0] != version:
            cached = (version, torch.cat([p.detach() for p in params], 0).contiguous())
            self.__dict__["_qkv_weight"] = cached
        return cached[1]

    def decodes_mixed(self, first: Tensor, position_device: Tensor | None) -> bool:
        """Whether ``decode`` can take its input as a depth mix (``mix=``)
        and make it inside the q|k|v projection's launch."""
        from . import hip_moe
        c = self.cfg
        return (self._hip(first) and position_device is not None and
                hip_moe.decode_qkv_supported(first.numel() // first.shape[-1], c.dim, c.n_heads,
                                             c.n_kv_heads, c.head_dim))

    def defers_sum(self, x: Tensor, position_device: Tensor | None,
                   cache: LocalKVCache) -> bool:
        """Whether decode(defer_sum=True) takes this input and cache: the HIP
        decode path at at most hip_moe.DEFER_MAX_TOKENS rows and within the
        shape limits of the per-head kernel and the pending mix, which
        returns the per-head contributions of the output projection instead
        of their sum."""
        if not (self._hip(x) and position_device is not None):
            return False
        from . import hip_moe
        c = self.cfg
        b = x.numel() // x.shape[-1]
        return hip_moe.decode_attention_heads_supported(
            b, x.shape[-1], c.n_heads, c.n_kv_heads, c.head_dim, cache.key.shape[2],
            c.window_size)

    def decode(self, x: Tensor | None, cache: LocalKVCache, position: int,
               addend: Tensor | None = None, defer_sum: bool = False,
               position_device: Tensor | None = None, mix: tuple | None = None,
               embed: tuple | None = None) -> Tensor:
        """One decode step; ``mix = (depth_module, sources, norm)`` in place
        of x gives the input as that depth mix + norm (see decodes_mixed).
        ``embed = (token_ids, embedding weight)`` with a one-source mix: that
        source is filled with the tokens' embedding rows by the same launch
        (hip_moe.decode_qkv)."""
        if embed is not None and mix is None:
            raise RuntimeError("an embedded decode input needs the one-source mix it fills")
        if mix is not None:
            if not self.decodes_mixed(mix[1][0], position_device):
                raise RuntimeError("this decode step cannot take its input as a depth mix")
            x = mix[1][0]  # shape, dtype and device of the input rows
        if x.shape[1] != 1:
            raise ValueError("decode expects one model position")
        c = self.cfg
        b = x.shape[0]
        if defer_sum and not self.defers_sum(x, position_device, cache):
            raise RuntimeError("deferred attention reduction is not supported for this input")
        if self._hip(x) and position_device is not None:
            # RoPE at the device position, then one kernel stores the new key
            # and value and attends over the window (parrot/model.py:239-262).
            from . import hip_moe
            cos, sin = _rope_tables(c, x.new_empty(0, dtype=torch.float32))
            if mix is not None:
                q, k, v = hip_moe.decode_qkv(None, self._packed_qkv(), cos, sin, c.n_heads,
                                             c.n_kv_heads, c.head_dim, position_device, mix=mix,
                                             embed=embed)
            elif self._fused_projections():
                q, k, v = hip_moe.proj_rope_qkv(x, self._qkv_fragments(), cos, sin, c.n_heads,
                                                c.n_kv_heads, c.head_dim,
                                                start_device=position_device)
            else:
                q, k, v = hip_moe.rope_qkv(F.linear(x, self._packed_qkv()), cos, sin, c.n_heads,
                                           c.n_kv_heads, c.head_dim, 0, False,
                                           start_device=position_device)
            if defer_sum:
                # Per-head contributions of the output projection; the caller
                # wraps them (with the addend) in a PendingResidual.
                return hip_moe.decode_attention_heads(q, k, v, cache.key, cache.value,
                                                      position_device, c.window_size,
                                                      c.head_dim ** -0.5, self.out.weight)
            y = hip_moe.decode_attention(q, k, v, cache.key, cache.value, position_device,
                                         c.window_size, c.head_dim ** -0.5)
            width = c.n_heads * c.head_dim
            # The GEMV beats the MFMA projection for one or two rows (measured
            # at b = 1 / 2 / 8: 0.525 -> 0.515, 0.559 -> 0.553, 0.730 -> 0.776 ms
            # per decode step).
            if b <= 2 and hip_moe.decode_linear_supported(b, width, c.dim):
                return hip_moe.decode_linear(y.view(b, 1, width), self.out.weight, addend)
            return self._project_out(y.view(b, 1, -1), addend)
        if self._hip(x):
            q, k, v = self._qkv(x, start=position)
        else:
            qw, kw = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
            q, k, v = F.linear(x, self._packed_qkv()).split((qw, kw, kw), dim=-1)
            q = _apply_rope(c, q.view(b, 1, c.n_heads, c.head_dim).transpose(1, 2), position)
            k = _apply_rope(c, k.view(b, 1, c.n_kv_heads, c.head_dim).transpose(1, 2), position)
            v = v.view(b, 1, c.n_kv_heads, c.head_dim).transpose(1, 2)
        cache.key[:, :, position:position + 1].copy_(k)
        cache.value[:, :, position:position + 1].copy_(v)
        lo = max(0, position - c.window_size + 1)
        y = F.scaled_dot_product_attention(
            q, cache.key[:, :, lo:position + 1], cache.value[:, :, lo:position + 1],
            enable_gqa=True)
        result = self.out(y.transpose(1, 2).reshape(b, 1, -1))
        return result if addend is None else addend + result


class GlobalMLA(nn.Module):
    """NoPE attention over a joint KV latent (reference parrot/model.py:331-432).

    Prefill expands the latent into heads; decode keeps only the latent and
    absorbs the key/value up-projections into the query and output maps."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        width = cfg.n_heads * cfg.head_dim
        self.q = nn.Linear(cfg.dim, width, bias=False)
        self.kv_down = nn.Linear(cfg.dim, cfg.kv_latent_dim, bias=False)
        self.k_up = nn.Linear(cfg.kv_latent_dim, width, bias=False)
        self.v_up = nn.Linear(cfg.kv_latent_dim, width, bias=False)
        self.out = nn.Linear(width, cfg.dim, bias=False)

    def forward(self, x: Tensor, addend: Tensor | None = None) -> Tensor:
        return self.prefill(x, addend)[0]

    def fuses_addend(self, x: Tensor) -> bool:
        """True when ``prefill(x, addend)`` folds the residual add into the
        output projection kernel."""
        return self.cfg.uses_hip and _hip_inference(x) and self._fused_projections()

    def _fused_projections(self) -> bool:
        from . import hip_moe
        c = self.cfg
        width, r = c.n_heads * c.head_dim, c.kv_latent_dim
        return (c.head_dim in hip_moe.ATTENTION_HEAD_DIMS and r % 8 == 0 and
                hip_moe.proj_supported(c.dim, width + r) and
                hip_moe.proj_supported(r, 2 * width) and hip_moe.proj_supported(width, c.dim))

    def defers_heads(self, x: Tensor) -> bool:
        """True when ``prefill_heads(x)`` applies (see LocalGQA)."""
        from . import hip_moe
        c = self.cfg
        return (self.fuses_addend(x) and
                hip_moe.attention_heads_out_supported(c.n_heads, c.head_dim, c.dim))

    def prefill_heads(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """``prefill(x)`` with the output projection deferred per head: (fp32
        contributions [b, t, H, dim], latent) (see LocalGQA.prefill_heads)."""
        from . import hip_moe
        b, t, _ = x.shape
        c = self.cfg
        width = c.n_heads * c.head_dim
        qkv = hip_moe.proj(x, self._fragments("q", "kv_down"), width + c.kv_latent_dim)
        q, latent = qkv[..., :width], qkv[..., width:]
        kf, vf = hip_moe.proj_kv_frag(latent, self._fragments("k_up", "v_up"), width, c.head_dim)
        q = q.view(b, t, c.n_heads, c.head_dim).transpose(1, 2)
        return hip_moe.causal_attention_frag_out(q, kf, vf, self._fragments("out"), c.dim,
                                                 kv_heads=c.n_heads,
                                                 scale=c.head_dim ** -0.5), latent

    def _fragments(self, *names: str) -> Tensor:
        """The named linears' weights, row-concatenated and packed."""
        from . import hip_moe
        return hip_moe.pack_linear(self, "_".join(names),
                                   tuple(getattr(self, n).weight for n in names))

    def prefill(self, x: Tensor, addend: Tensor | None = None) -> tuple[Tensor, Tensor]:
        """(out(attention(x)) [+ addend], latent) over the whole sequence."""
        b, t, _ = x.shape
        c = self.cfg
        width = c.n_heads * c.head_dim

        def heads(y):
            return y.view(b, t, c.n_heads, c.head_dim).transpose(1, 2)

        if c.uses_hip and _hip_inference(x) and self._fused_projections():
            # Three projection kernels around one attention kernel: q with
            # kv_down, then k_up with v_up writing K and V in the attention
            # kernel's fragment order, then the output projection.
            from . import hip_moe
            qkv = hip_moe.proj(x, self._fragments("q", "kv_down"), width + c.kv_latent_dim)
            q, latent = qkv[..., :width], qkv[..., width:]
            kf, vf = hip_moe.proj_kv_frag(latent, self._fragments("k_up", "v_up"), width,
                                          c.head_dim)
            y = hip_moe.causal_attention_frag(heads(q), kf, vf, kv_heads=c.n_heads,
                                              scale=c.head_dim ** -0.5)
            return hip_moe.proj(y, self._fragments("out"), c.dim, addend=addend), latent
        latent = self.kv_down(x)
        if c.uses_hip and _hip_inference(x):
            from . import hip_moe
            if c.head_dim in hip_moe.ATTENTION_HEAD_DIMS:
                # Values produced transposed, [b, H * d, keys], by one GEMM.
                latent_t = F.pad(latent.transpose(1, 2), (0, hip_moe.padded_keys(t) - t))
                vt = torch.matmul(self.v_up.weight, latent_t).view(
                    b, c.n_heads, c.head_dim, -1)
                y = hip_moe.causal_attention(heads(self.q(x)), heads(self.k_up(latent)), vt=vt,
                                             scale=c.head_dim ** -0.5)
                result = self.out(y)
                return (result if addend is None else addend + result), latent
        y = F.scaled_dot_product_attention(
            heads(self.q(x)), heads(self.k_up(latent)), heads(self.v_up(latent)),
            is_causal=True)
        result = self.out(y.transpose(1, 2).reshape(b, t, -1))
        return (result if addend is None else addend + result), latent

    def _absorbed(self) -> tuple[Tensor, Tensor]:
        """(W_q absorbed with k_up [H*L, dim], v_up absorbed with out [dim, H*L])."""
        cached = self.__dict__.get("_absorbed_weights")
        if cached is not None and not torch.is_grad_enabled() and not self.training:
            return cached[1]
        c = self.cfg
        params = (self.q.weight, self.k_up.weight, self.v_up.weight, self.out.weight)
        version = tuple((p._version, p.device, p.dtype, p.data_ptr()) for p in params)
        if cached is None or cached[0] != version:
            with torch.no_grad():
                wq = self.q.weight.detach().float().view(c.n_heads, c.head_dim, c.dim)
                wk = self.k_up.weight.detach().float().view(c.n_heads, c.head_dim, c.kv_latent_dim)
                wv = self.v_up.weight.detach().float().view(c.n_heads, c.head_dim, c.kv_latent_dim)
                wo = self.out.weight.detach().float().view(c.dim, c.n_heads, c.head_dim)
                # q_latent[h, l] = sum_d k_up[h, d, l] q[h, d]
                absorbed_q = torch.matmul(wk.transpose(1, 2), wq).reshape(
                    c.n_heads * c.kv_latent_dim, c.dim)
                # out[m] = sum_{h, l} (sum_d out[m, h, d] v_up[h, d, l]) ctx[h, l]
                absorbed_o = torch.matmul(wo.permute(1, 0, 2), wv).permute(1, 0, 2).reshape(
                    c.dim, c.n_heads * c.kv_latent_dim)
                dtype = self.q.weight.dtype
                cached = (version, (absorbed_q.to(dtype).contiguous(),
                                    absorbed_o.to(dtype).contiguous()))
            self.__dict__["_absorbed_weights"] = cached
        return cached[1]

    def _absorbed_f32(self) -> tuple[Tensor, Tensor]:
        """fp32 copies of the absorbed maps, cached with them."""
        pair = self._absorbed()
        cached = self.__dict__.get("_absorbed_f32_weights")
        if cached is None or cached[0] is not pair:
            cached = (pair, (pair[0].float(), pair[1].float()))
            self.__dict__["_absorbed_f32_weights"] = cached
        return cached[1]

    def decodes_mixed(self, first: Tensor, position_device: Tensor | None) -> bool:
        """Whether ``decode`` can take its input as a depth mix (``mix=``)
        and make it inside the projections' launch."""
        from . import hip_moe
        c = self.cfg
        b = first.numel() // first.shape[-1]
        return (c.uses_hip and _hip_inference(first) and position_device is not None and
                c.dim <= 1024 and self.kv_down.weight.dtype == first.dtype and
                hip_moe.mla_decode_supported(b, c.dim, c.n_heads * c.kv_latent_dim))

    def decode(self, x: Tensor | None, cache: MLALatentCache, position: int,
               addend: Tensor | None = None, defer_sum: bool = False,
               position_device: Tensor | None = None, mix: tuple | None = None) -> Tensor:
        """One decode step; ``mix = (depth_module, sources, norm)`` in place
        of x gives the input as that depth mix + norm (see decodes_mixed)."""
        if mix is not None:
            if not self.decodes_mixed(mix[1][0], position_device):
                raise RuntimeError("this decode step cannot take its input as a depth mix")
            x = mix[1][0]  # shape, dtype and device of the input rows
        if x.shape[1] != 1:
            raise ValueError("decode expects one model position")
        if defer_sum:
            raise RuntimeError("deferred attention reduction is not supported on this backend")
        c = self.cfg
        b = x.shape[0]
        if c.uses_hip and _hip_inference(x) and position_device is not None:
            # One kernel stores the new latent and attends over the latent
            # cache at the device position (parrot/model.py:399-432).
            from . import hip_moe
            width = c.n_heads * c.kv_latent_dim
            if (hip_moe.mla_decode_supported(b, c.dim, width)
                    and self.kv_down.weight.dtype == x.dtype):
                # Three launches: projections, latent attention, output map.
                absorbed_q, absorbed_o = self._absorbed()
                q_latent, latent = hip_moe.mla_decode_in(None if mix is not None else x,
                                                         absorbed_q, self.kv_down.weight,
                                                         mix=mix)
                context = hip_moe.decode_attention_latent(
                    q_latent, latent, cache.latent, position_device, c.n_heads,
                    c.head_dim ** -0.5)
                return hip_moe.mla_decode_out(context, absorbed_o, addend)
            absorbed_q, absorbed_o = self._absorbed_f32()
            context = hip_moe.decode_attention_latent(
                F.linear(x.float(), absorbed_q), self.kv_down(x), cache.latent, position_device,
                c.n_heads, c.head_dim ** -0.5)
            result = F.linear(context.view(b, 1, -1), absorbed_o).to(x.dtype)
            return result if addend is None else addend + result
        absorbed_q, absorbed_o = self._absorbed()
        cache.latent[:, position:position + 1].copy_(self.kv_down(x))
        latent = cache.latent[:, :position + 1].float()
        q_latent = F.linear(x.float(), absorbed_q.float()).view(
            b, 1, c.n_heads, c.kv_latent_dim).transpose(1, 2)
        per_head = latent[:, None].expand(-1, c.n_heads, -1, -1)
        context = F.scaled_dot_product_attention(q_latent, per_head, per_head,
                                                 scale=c.head_dim ** -0.5)
        context = context.transpose(1, 2).reshape(b, 1, c.n_heads * c.kv_latent_dim)
        result = F.linear(context, absorbed_o.float()).to(x.dtype)
        return result if addend is None else addend + result


class SwiGLU(nn.Module):
    def __init__(self, dim: int, intermediate: int):
        super().__init__()
        self.gate = nn.Linear(dim, intermediate, bias=False)
        self.up = nn.Linear(dim, intermediate, bias=False)
        self.down = nn.Linear(intermediate, dim, bias=False)

    def forward(self, x: Tensor) -> Tensor:
        return self.down(F.silu(self.gate(x)) * self.up(x))


class MoE(nn.Module):
    """Top-k routed SwiGLU experts plus one shared expert
    (reference parrot/model.py:463-607)."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.router = nn.Linear(cfg.dim, cfg.n_experts, bias=False)
        self.experts = nn.ModuleList(
            [SwiGLU(cfg.dim, cfg.expert_dim) for _ in range(cfg.n_experts)])
        self.shared = SwiGLU(cfg.dim, cfg.shared_expert_dim)

    def _hip_route_applies(self, x: Tensor) -> bool:
        return (self.cfg.moe_backend == "grouped_hip" and _hip_inference(x) and
                self.cfg.top_k == 2 and self.cfg.n_experts <= 32)

    def _torch_route(self, flat: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        # Router projection and softmax in fp32 with autocast off.
        with torch.autocast(device_type=flat.device.type, enabled=False):
            probs = F.linear(flat.float(), self.router.weight.float()).softmax(-1)
        weights, indices = probs.topk(self.cfg.top_k, dim=-1)
        return probs, weights / weights.sum(-1, keepdim=True), indices

    def _torch_experts(self, flat: Tensor, weights: Tensor, indices: Tensor) -> Tensor:
        result = self.shared(flat)
        for e, expert in enumerate(self.experts):
            rows, slots = torch.where(indices == e)
            if rows.numel():
                contribution = expert(flat[rows]) * weights[rows, slots, None].to(result.dtype)
                result = result.index_add(0, rows, contribution)
        return result

    def forward(self, x: Tensor) -> tuple[Tensor, Tensor | None, Tensor | None]:
        flat = x.reshape(-1, x.shape[-1])
        route_counts = None
        grouping = None
        if self._hip_route_applies(x):
            from . import hip_moe
            routed = hip_moe.route(self, flat, self.cfg.collect_router_stats)
            probs, weights, indices = routed.probabilities, routed.weights, routed.indices
            grouping = routed.grouping
            route_counts = grouping.counts
        else:
            probs, weights, indices = self._torch_route(flat)
        if self.cfg.moe_backend == "grouped_hip":
            from . import hip_moe
            result = hip_moe.grouped_hip_experts(self, flat, indices, weights,
                                                 grouping=grouping)
        else:
            result = self._torch_experts(flat, weights, indices)
        if not self.cfg.collect_router_stats:
            return result.view_as(x), None, None
        if route_counts is not None:
            counts = route_counts.float()
        else:
            flat_idx = indices.flatten()
            counts = torch.zeros(self.cfg.n_experts, device=indices.device,
                                 dtype=torch.float32).scatter_add_(
                0, flat_idx, torch.ones(flat_idx.shape, device=indices.device,
                                        dtype=torch.float32))
        utilization = counts / indices.numel()
        aux = self.cfg.n_experts * (utilization * probs.mean(0)).sum()
        return result.view_as(x), aux, utilization.detach()

    def inference(self, x: Tensor, *, direct: bool, addend: Tensor | None = None,
                  defer_sum: bool = False) -> Tensor:
        """Inference without router statistics.  On the HIP backend the
        addend (an open AttnRes partial sum) is folded into the combine
        kernel; inputs of at most 16 rows (decode steps) run the fused
        two-launch decode MoE, larger ones route + grouped experts with tiles
        chosen by size (so ``direct`` needs no separate handling)."""
        if defer_sum:
            raise ValueError("deferred MoE reduction is not supported on this backend")
        if not self._hip_route_applies(x):
            result = self.forward(x)[0]
            return result if addend is None else addend + result
        from . import hip_moe
        flat = x.reshape(-1, x.shape[-1])
        if flat.shape[0] <= hip_moe.DECODE_MAX_TOKENS:
            # Decode-sized inputs: the whole layer in two launches.
            return hip_moe.decode_experts(self, flat, addend=addend)[0].view_as(x)
        routed = hip_moe.route_for_experts(self, flat)
        result = hip_moe.grouped_hip_experts(self, flat, routed.indices, routed.weights,
                                             addend=addend, grouping=routed.grouping,
                                             route_blocks=routed.blocks)
        return result.view_as(x)


    def routes_in_depth_mix(self, x: Tensor) -> bool:
        """Whether this layer's input depth mix also computes its top-2 route
        (hip_moe.depth_mix_norm_route): the grouped HIP path at sizes whose
        gate/up launch groups the indices itself, where the separate route
        and grouping launches are pure latency."""
        if not (self._hip_route_applies(x) and self.cfg.depth_backend == "hip"):
            return False
        from . import hip_moe
        tokens = x.numel() // x.shape[-1]
        return (tokens > hip_moe.DECODE_MAX_TOKENS and
                hip_moe.groups_in_kernel(self, tokens, x.shape[-1]))

    def inference_then_mix(self, x: Tensor, *, addend: Tensor | None, depth: "DepthMix",
                           sources: list[Tensor], output_norm: "RMSNorm",
                           routed=None) -> tuple[Tensor, Tensor]:
        """``inference(x, addend=addend)`` and the next module's input,
        ``depth.normalized(sources + [result], output_norm)``; on the grouped
        HIP path the combine and that depth mix are one kernel.  ``routed``:
        x's top-2 route when its depth mix already computed it."""
        from . import hip_moe
        flat = x.reshape(-1, x.shape[-1])
        if (self._hip_route_applies(x) and flat.shape[0] > hip_moe.DECODE_MAX_TOKENS and
                depth.cfg.depth_backend == "hip" and
                len(sources) < hip_moe.MAX_DEPTH_SOURCES):
            if routed is None:
                routed = hip_moe.route_for_experts(self, flat)
            result, mixed = hip_moe.grouped_hip_experts(
                self, flat, routed.indices, routed.weights, addend=addend,
                grouping=routed.grouping, then_mix=(depth, sources, output_norm),
                route_blocks=routed.blocks)
            return result.view_as(x), mixed.view_as(x)
        result = self.inference(x, direct=False, addend=addend)
        return result, depth.normalized(sources + [result], output_norm)


class Block(nn.Module):
    def __init__(self, cfg: ModelConfig, index: int):
        super().__init__()
        is_global = (index + 1) % cfg.global_every == 0
        self.attention = GlobalMLA(cfg) if is_global else LocalGQA(cfg)
        self.moe = MoE(cfg)
        self.attention_norm = RMSNorm(cfg.dim, cfg.norm_eps, cfg.uses_hip)
        self.moe_norm = RMSNorm(cfg.dim, cfg.norm_eps, cfg.uses_hip)

    def attend(self, x: Tensor) -> Tensor:
        return self.attention(self.attention_norm(x))

    def feedforward(self, x: Tensor):
        return self.moe(self.moe_norm(x))

    def feedforward_inference(self, x: Tensor, *, direct: bool) -> Tensor:
        return self.moe.inference(self.moe_norm(x), direct=direct)


class _AttnRes:
    """Block AttnRes residual stream: completed block sums plus the open
    partial sum of the current block (reference parrot/model.py:680-710)."""

    def __init__(self, embedded: Tensor, block_size: int):
        self.completed = [embedded]
        self.partial: Tensor | None = None
        self.block_size = block_size
        self.modules = 0

    def sources(self) -> list[Tensor]:
        return self.completed if self.partial is None else self.completed + [self.partial]

    def close(self, summed: Tensor) -> None:
        """Record ``partial + delta`` (already summed) for the next module."""
        self.partial = summed
        self.modules += 1
        if self.modules % self.block_size == 0:
            self.completed.append(summed)
            self.partial = None

    def push(self, delta: Tensor) -> None:
        self.close(delta if self.partial is None else self.partial + delta)


class Parrot(nn.Module):
    def __init__(self, cfg: ModelConfig = ModelConfig()):
        super().__init__()
        self.config = cfg
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.dim)
        self.blocks = nn.ModuleList([Block(cfg, i) for i in range(cfg.n_layers)])
        self.depth_mix = nn.ModuleList(
            [DepthMix(cfg) for _ in range(2 * cfg.n_layers + 1)]
            if cfg.residual == "attnres" else [])
        self.final_norm = RMSNorm(cfg.dim, cfg.norm_eps, cfg.uses_hip)
        # The vocabulary head is tied to embedding.weight.
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module):
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, std=0.02)

    # -- helpers -------------------------------------------------------------

    def _embedded(self, input_ids: Tensor, bag_size: int = 1,
                  stat_zeros: Tensor | None = None) -> tuple[Tensor, Tensor | None]:
        """The embedding rows (parrot/model.py:679) and, where the HIP path
        makes it in the same launch, the first module's input (else None);
        ``stat_zeros`` is zero-filled by that launch."""
        if not self._embeds_first_mix(input_ids, bag_size):
            x = self.embedding(input_ids)
            if bag_size > 1:
                b, source_len = input_ids.shape
                x = x.reshape(b, source_len // bag_size, bag_size, -1).mean(2)
            return x, None
        from . import hip_moe
        weight = self.embedding.weight
        if not torch.cuda.is_current_stream_capturing():
            # The launch clamps ids outside the table (a graph replay has no
            # error channel); an eager call raises as nn.Embedding does.
            if bool(((input_ids < 0) | (input_ids >= weight.shape[0])).any()):
                raise IndexError(f"token id out of range of the {weight.shape[0]}-row embedding")
        return hip_moe.embed_depth_mix_norm(input_ids, weight, self.depth_mix[0],
                                            self.blocks[0].attention_norm, stat_zeros)

    def _embeds_first_mix(self, input_ids: Tensor, bag_size: int) -> bool:
        """The HIP forward's first launch gathers the embedding rows and makes
        the first module's input (AttnRes, one token per position)."""
        cfg = self.config
        return (bag_size == 1 and cfg.residual == "attnres" and cfg.depth_backend == "hip" and
                len(self.blocks) > 0 and input_ids.dtype == torch.int64 and
                input_ids.device == self.embedding.weight.device and
                _hip_inference(self.embedding.weight))

    def _head(self, normed: Tensor) -> Tensor:
        """Tied vocabulary head (reference parrot/model.py:714-715).  On the
        HIP backend the logits come out in fp32, never rounded to bf16: a
        bf16 rounding of ~0.5-magnitude logits (ulp 2^-8) ties or swaps
        near-equal top logits, the head's share of greedy-argmax
        disagreement with the fp32 reference."""
        if self.config.uses_hip and _hip_inference(normed):
            from . import hip_moe
            return hip_moe.vocab_logits(normed, self.embedding.weight)
        return F.linear(normed, self.embedding.weight)

    def _mixed_input(self, stream: _AttnRes | None, x: Tensor, index: int,
                     norm: RMSNorm) -> Tensor:
        """Normalised input of module ``index``: RMSNorm of the depth mix
        (AttnRes) or of the running residual (standard)."""
        if stream is None:
            return norm(x)
        return self.depth_mix[index].normalized(stream.sources(), norm)

    def _moe_input(self, block: Block, stream: _AttnRes | None, x: Tensor, index: int):
        """MoE module ``index``'s normalised input and, when its depth mix
        kernel also routes it (MoE.routes_in_depth_mix, with the MoE about
        to close the open partial sum), its top-2 route; else (input, None)."""
        if (stream is not None and stream.partial is not None and
                not self.config.collect_router_stats):
            sources = stream.sources()
            first = sources[0]
            pending = stream.partial if isinstance(stream.partial, PendingResidual) else None
            if block.moe.routes_in_depth_mix(first):
                from . import hip_moe
                if pending is None:
                    return hip_moe.depth_mix_norm_route(self.depth_mix[index], sources,
                                                        block.moe_norm, block.moe)
                # The deferred attention output is summed and written inside
                # the mix; it is then the open partial sum the MoE closes.
                resolved = torch.empty_like(first)
                placeholder = pending.base if pending.base is not None else first
                contributions = pending.contributions.view(-1, *pending.contributions.shape[-2:])
                h, routed = hip_moe.depth_mix_norm_route(
                    self.depth_mix[index], sources[:-1] + [placeholder], block.moe_norm,
                    block.moe, pending=(contributions, pending.base, resolved))
                stream.partial = resolved
                return h, routed
            if pending is not None:  # _defers_attention_heads checked the same predicate
                raise RuntimeError("a deferred attention output needs the fused MoE input mix")
        return self._mixed_input(stream, x, index, block.moe_norm), None

    def _fuses_decode_moe(self, block: Block, first: Tensor) -> bool:
        """Whether a decode step's MoE module makes its input's depth mix +
        norm inside the fused decode MoE's launches."""
        if self.config.depth_backend != "hip" or not block.moe._hip_route_applies(first):
            return False
        from . import hip_moe
        tokens, dim = first.numel() // first.shape[-1], first.shape[-1]
        return tokens <= hip_moe.DECODE_MAX_TOKENS and dim <= 1024

    def _defers_attention(self, block: Block, stream: _AttnRes, index: int,
                          state: GenerationState) -> bool:
        """Whether attention module ``index`` of a decode step leaves its
        output's sum to the MoE's input mix: local layers on the HIP path at
        at most hip_moe.DEFER_MAX_TOKENS rows, when the module does not close
        a depth block (its output is then read by that mix alone)."""
        first = stream.sources()[0]
        return (isinstance(block.attention, LocalGQA) and
                (index + 1) % self.config.depth_block_size != 0 and
                block.attention.defers_sum(first, state.position_device,
                                           state.layers[index // 2]) and
                self._fuses_decode_moe(block, first))

    @staticmethod
    def _resolve(pending: PendingResidual, dtype: torch.dtype) -> Tensor:
        """``base + round(sum of the contributions)`` in ``dtype`` (the
        pending item's value) with torch ops, for consumers that do not
        resolve it themselves."""
        delta = pending.contributions.sum(1, keepdim=True).to(dtype)
        if pending.base is None:
            return delta
        return (pending.base.float() + delta.float()).to(dtype)

    def _decode_moe(self, block: Block, stream: _AttnRes, x: Tensor, index: int) -> Tensor:
        """MoE module ``index`` of a decode step, closing the open partial sum
        (``partial + delta``).  On the HIP path its input's depth mix + norm
        runs inside the fused decode MoE's launches, resolving a pending
        attention output there too."""
        sources = stream.sources()
        first = sources[0]
        pending = stream.partial if isinstance(stream.partial, PendingResidual) else None
        if self._fuses_decode_moe(block, first):
            from . import hip_moe
            mix_depth = self.depth_mix[index]
            if pending is None:
                out = hip_moe.decode_experts(
                    block.moe, None, addend=stream.partial,
                    mix=(mix_depth, sources, block.moe_norm))[0]
            else:
                resolved = torch.empty_like(first)
                placeholder = pending.base if pending.base is not None else first
                out = hip_moe.decode_experts(
                    block.moe, None, addend=resolved,
                    mix=(mix_depth, sources[:-1] + [placeholder], block.moe_norm),
                    pending=(pending.contributions, pending.base, resolved))[0]
            return out.view_as(first)
        if pending is not None:
            stream.partial = self._resolve(pending, first.dtype)
        h = self._mixed_input(stream, x, index, block.moe_norm)
        return block.moe.inference(h, direct=True, addend=stream.partial)

    def _moe_closing(self, block: Block, h: Tensor, stream: _AttnRes, index: int,
                     next_norm: RMSNorm, routed=None) -> Tensor:
        """Close MoE module ``index`` (fused addend) and return the input of
        module ``index + 1``: its depth mix normalised by ``next_norm``, made
        by the MoE's combine kernel on the HIP path.  ``routed``: h's top-2
        route when its depth mix computed it."""
        older = list(stream.completed)  # the sources after closing: older + [result]
        result, mixed = block.moe.inference_then_mix(
            h, addend=stream.partial, depth=self.depth_mix[index + 1], sources=older,
            output_norm=next_norm, routed=routed)
        stream.close(result)
        return mixed

    def _defers_attention_heads(self, block: Block, h: Tensor, stream: _AttnRes | None,
                                index: int) -> bool:
        """Whether attention module ``index`` of a whole-sequence forward
        leaves its output projection's sum over heads to the MoE's input mix
        (hip_moe.depth_mix_norm_route with ``pending``): that mix must be the
        fused route mix, and the module must not close a depth block (its
        output is then read by that mix alone before the MoE adds to it)."""
        cfg = self.config
        return (stream is not None and not cfg.collect_router_stats and
                (index + 1) % cfg.depth_block_size != 0 and
                block.attention.defers_heads(h) and
                block.moe.routes_in_depth_mix(stream.sources()[0]))

    @staticmethod
    def _fuse_attention_addend(block: Block, h: Tensor, stream: _AttnRes | None) -> bool:
        """Fold ``partial + delta`` into the attention output projection (HIP only)."""
        return stream is not None and stream.partial is not None and \
            block.attention.fuses_addend(h)

    def _fuse_moe_addend(self, block: Block, h: Tensor, stream: _AttnRes | None) -> bool:
        """Fold ``partial + delta`` into the MoE combine kernel (HIP only)."""
        return (stream is not None and stream.partial is not None and
                not self.config.collect_router_stats and block.moe._hip_route_applies(h))

    # -- training / full-sequence forward ------------------------------------

    def forward(self, input_ids: Tensor, labels: Tensor | None = None, *,
                bag_size: int = 1, supervised_logits_only: bool = False) -> ModelOutput:
        """Unpadded streams; labels are UNSHIFTED source-token ids or -100.

        bag_size=1: position i predicts token i+1.  bag_size>1: the mean
        embedding of bag i predicts every token of bag i+1."""
        cfg = self.config
        if input_ids.ndim != 2 or input_ids.numel() == 0:
            raise ValueError("input_ids must be a nonempty [batch, source_tokens] tensor")
        if not isinstance(bag_size, int) or bag_size < 1 or input_ids.shape[1] % bag_size:
            raise ValueError("source_tokens must be divisible by positive integer bag_size")
        b, source_len = input_ids.shape
        t = source_len // bag_size
        if t > cfg.max_seq_len:
            raise ValueError("Input exceeds max_seq_len model positions")
        if labels is not None and (labels.shape != input_ids.shape or t < 2):
            raise ValueError("labels must match input_ids and contain at least two model positions")
        if supervised_logits_only and labels is None:
            raise ValueError("supervised_logits_only requires labels")

        stat_zeros = None
        if self._embeds_first_mix(input_ids, bag_size) and not cfg.collect_router_stats:
            stat_zeros = torch.empty((1 + cfg.n_layers * cfg.n_experts,), dtype=torch.float32,
                                     device=self.embedding.weight.device)
        # pending: the next module's input (the first module's from the
        # embedding launch, then each made by the previous MoE's combine)
        x, pending = self._embedded(input_ids, bag_size, stat_zeros)
        stream = _AttnRes(x, cfg.depth_block_size) if cfg.residual == "attnres" else None
        aux_losses, utilization = [], []
        remat = cfg.checkpoint_modules and self.training and torch.is_grad_enabled()
        index = 0
        for bi, block in enumerate(self.blocks):
            h = pending if pending is not None else \
                self._mixed_input(stream, x, index, block.attention_norm)
            pending = None
            if not remat and self._defers_attention_heads(block, h, stream, index):
                # the MoE's input mix sums the heads (and adds the partial sum)
                stream.close(PendingResidual(stream.partial, block.attention.prefill_heads(h)[0]))
            elif not remat and self._fuse_attention_addend(block, h, stream):
                stream.close(block.attention(h, addend=stream.partial))
            else:
                delta = (checkpoint(block.attention, h, use_reentrant=False) if remat
                         else block.attention(h))
                if stream is None:
                    x = x + delta
                else:
                    stream.push(delta)
            index += 1

            h, routed = self._moe_input(block, stream, x, index)
            if self._fuse_moe_addend(block, h, stream):
                last = bi + 1 == len(self.blocks)
                pending = self._moe_closing(
                    block, h, stream, index,
                    self.final_norm if last else self.blocks[bi + 1].attention_norm, routed)
            else:
                delta, aux, usage = (checkpoint(block.moe, h, use_reentrant=False) if remat
                                     else block.moe(h))
                if cfg.collect_router_stats:
                    aux_losses.append(aux)
                    utilization.append(usage)
                if stream is None:
                    x = x + delta
                else:
                    stream.push(delta)
            index += 1
        if pending is not None:
            # The last MoE's combine produced final_norm(depth_mix[-1](...)).
            normed = pending[:, :-1] if supervised_logits_only else pending
        else:
            if stream is not None:
                x = self.depth_mix[-1](stream.sources())
            # Loss-only callers can skip the last position's projection exactly.
            normed = self.final_norm(x[:, :-1] if supervised_logits_only else x)
        logits = self._head(normed)

        if cfg.collect_router_stats:
            aux_loss = torch.stack(aux_losses).mean()
            expert_utilization = torch.stack(utilization)
        else:
            # one zero fill for both (views of one buffer; on the HIP path the
            # first launch filled it)
            zeros = stat_zeros if stat_zeros is not None else \
                x.new_zeros((1 + cfg.n_layers * cfg.n_experts,), dtype=torch.float32)
            aux_loss = zeros[0]
            expert_utilization = zeros[1:].view(cfg.n_layers, cfg.n_experts)
        lm_loss = loss = None
        if labels is not None:
            targets = labels.reshape(b, t, bag_size)[:, 1:]
            loss_logits = (logits if supervised_logits_only else logits[:, :-1]).float()
            valid = targets != -100
            picked = loss_logits.gather(-1, targets.masked_fill(~valid, 0))
            lse = torch.logsumexp(loss_logits, dim=-1)
            total = (lse * valid.sum(-1) - (picked * valid).sum(-1)).sum()
            lm_loss = total / valid.sum().clamp_min(1)
            loss = lm_loss + cfg.aux_loss_weight * aux_loss
        return ModelOutput(logits, loss, lm_loss, aux_loss, expert_utilization)

    # -- incremental generation ----------------------------------------------

    @torch.inference_mode()
    def prefill(self, input_ids: Tensor) -> tuple[Tensor, GenerationState]:
        """Run the prompt once; return next-token logits and the KV state."""
        cfg = self.config
        if self.training:
            raise RuntimeError("prefill requires model.eval()")
        if input_ids.ndim != 2 or input_ids.shape[1] < 1:
            raise ValueError("input_ids must be nonempty [batch, positions]")
        b, t = input_ids.shape
        if t > cfg.max_seq_len:
            raise ValueError("Prompt exceeds max_seq_len")
        # pending: the next module's input (the first module's from the
        # embedding launch, then each made by the previous MoE's combine)
        x, pending = self._embedded(input_ids)
        stream = _AttnRes(x, cfg.depth_block_size) if cfg.residual == "attnres" else None
        caches: list[LocalKVCache | MLALatentCache] = []
        index = 0
        for bi, block in enumerate(self.blocks):
            h = pending if pending is not None else \
                self._mixed_input(stream, x, index, block.attention_norm)
            pending = None
            defer = self._defers_attention_heads(block, h, stream, index)
            fuse = not defer and self._fuse_attention_addend(block, h, stream)
            addend = stream.partial if fuse else None
            local = isinstance(block.attention, LocalGQA)
            if defer:
                # as in forward: the MoE's input mix sums the heads
                if local:
                    delta, key, value = block.attention.prefill_heads(h, need_kv=True)
                else:
                    delta, latent = block.attention.prefill_heads(h)
                delta = PendingResidual(stream.partial, delta)
            elif local:
                delta, key, value = block.attention.prefill(h, addend)
            else:
                delta, latent = block.attention.prefill(h, addend)
            if local:
                shape = (b, cfg.n_kv_heads, cfg.max_seq_len, cfg.head_dim)
                cache = LocalKVCache(key.new_empty(shape), value.new_empty(shape))
                cache.key[:, :, :t].copy_(key)
                cache.value[:, :, :t].copy_(value)
            else:
                cache = MLALatentCache(latent.new_empty((b, cfg.max_seq_len, cfg.kv_latent_dim)))
                cache.latent[:, :t].copy_(latent)
            caches.append(cache)
            if fuse or defer:
                stream.close(delta)
            elif stream is None:
                x = x + delta
            else:
                stream.push(delta)
            index += 1

            h, routed = self._moe_input(block, stream, x, index)
            if stream is not None and stream.partial is not None and \
                    block.moe._hip_route_applies(h):
                last = bi + 1 == len(self.blocks)
                pending = self._moe_closing(
                    block, h, stream, index,
                    self.final_norm if last else self.blocks[bi + 1].attention_norm, routed)
            else:
                delta = block.moe.inference(h, direct=False)
                if stream is None:
                    x = x + delta
                else:
                    stream.push(delta)
            index += 1
        if pending is not None:
            normed = pending[:, -1:]  # final_norm(depth_mix[-1](...)) from the last combine
        else:
            if stream is not None:
                x = self.depth_mix[-1](stream.sources())
            normed = self.final_norm(x[:, -1:])
        logits = self._head(normed)
        position_device = None
        if cfg.uses_hip and _hip_inference(normed):
            position_device = torch.full((1,), t, dtype=torch.int32, device=logits.device)
        return logits, GenerationState(caches, t, b, position_device)

    def _decode_embedding(self, input_ids: Tensor,
                          state: GenerationState) -> tuple[Tensor, tuple | None]:
        """The decode step's embedding rows (parrot/model.py:830), or, when the
        first layer's q|k|v launch mixes its input on the HIP path, an unfilled
        row buffer and the (ids, weight) that launch gathers it from."""
        cfg = self.config
        first = self.blocks[0].attention if self.blocks else None
        if (cfg.residual == "attnres" and cfg.depth_backend == "hip" and
                isinstance(first, LocalGQA) and input_ids.is_cuda and
                state.position_device is not None and input_ids.dtype == torch.int64):
            weight = self.embedding.weight
            x = torch.empty((input_ids.shape[0], 1, cfg.dim), dtype=weight.dtype,
                            device=input_ids.device)
            if first.decodes_mixed(x, state.position_device):
                # The launch clamps ids outside the table to its nearest row
                # (a graph replay has no error channel).  An eager step checks
                # them first and raises as nn.Embedding does.
                if not torch.cuda.is_current_stream_capturing():
                    bad = (input_ids < 0) | (input_ids >= weight.shape[0])
                    if bool(bad.any()):
                        raise IndexError("decode_step token id out of range of the "
                                         f"{weight.shape[0]}-row embedding")
                return x, (input_ids, weight)
        return self.embedding(input_ids), None

    @torch.inference_mode()
    def decode_step(self, input_ids: Tensor, state: GenerationState, *,
                    _next_token_only: bool = False,
                    _out: Tensor | None = None) -> tuple[Tensor, GenerationState]:
        """Append one token per sequence to an existing generation state.
        ``_out`` (with ``_next_token_only``): an int64 [batch, 1] tensor the
        greedy tokens are written into and returned as."""
        cfg = self.config
        if self.training:
            raise RuntimeError("decode_step requires model.eval()")
        if input_ids.shape != (state.batch_size, 1):
            raise ValueError("decode_step input must be [cached batch, 1]")
        if state.position >= cfg.max_seq_len:
            raise ValueError("Generation state has reached max_seq_len")
        if len(state.layers) != cfg.n_layers:
            raise ValueError("Generation state does not match model depth")
        x, embed = self._decode_embedding(input_ids, state)
        stream = _AttnRes(x, cfg.depth_block_size) if cfg.residual == "attnres" else None
        index = 0
        for block, cache in zip(self.blocks, state.layers):
            addend = stream.partial if stream is not None else None
            if isinstance(block.attention, LocalGQA):
                if not isinstance(cache, LocalKVCache):
                    raise ValueError("Local attention received an MLA cache")
            elif not isinstance(cache, MLALatentCache):
                raise ValueError("MLA attention received a local cache")
            if (stream is not None and self.config.depth_backend == "hip" and
                    block.attention.decodes_mixed(stream.sources()[0], state.position_device)):
                # The input's depth mix + norm runs inside the q|k|v launch
                # (the first layer's also gathers the embedding rows).
                mix = (self.depth_mix[index], stream.sources(), block.attention_norm)
                extra = {"embed": embed} if index == 0 and embed is not None else {}
                if self._defers_attention(block, stream, index, state):
                    # The output projection's sum over heads is left to the
                    # MoE's input mix (the reference's PendingResidual).
                    delta = block.attention.decode(
                        None, cache, state.position, defer_sum=True,
                        position_device=state.position_device, mix=mix, **extra)
                    out = PendingResidual(addend, delta)
                else:
                    out = block.attention.decode(
                        None, cache, state.position, addend=addend,
                        position_device=state.position_device, mix=mix, **extra)
            else:
                h = self._mixed_input(stream, x, index, block.attention_norm)
                out = block.attention.decode(h, cache, state.position, addend=addend,
                                             position_device=state.position_device)
            if stream is None:
                x = x + out
            else:
                stream.close(out)  # out = partial + delta
            index += 1

            if stream is not None:
                stream.close(self._decode_moe(block, stream, x, index))
            else:
                x = x + block.feedforward_inference(x, direct=True)
            index += 1
        if stream is not None:
            h = self.depth_mix[-1].normalized(stream.sources(), self.final_norm)
        else:
            h = self.final_norm(x)
        advanced = False
        if _next_token_only and state.position_device is not None and h.shape[0] <= 16:
            # Greedy token straight from fp32 logits, never materialised
            # (cf. vocab_argmax_partials/reduce_bf16, moe_bf16.metal:1541-1621);
            # the same launch advances the device position.
            from . import hip_moe
            output = hip_moe.vocab_argmax(h, self.embedding.weight, advance=state.position_device,
                                          out=_out)
            advanced = True
        else:
            logits = self._head(h)
            output = logits.argmax(-1) if _next_token_only else logits
            if _next_token_only and _out is not None:
                output = _out.copy_(output)
        state.position += 1
        if state.position_device is not None and not advanced:
            state.position_device.add_(1)
        return output, state

    @torch.inference_mode()
    def decode_next(self, input_ids: Tensor,
                    state: GenerationState) -> tuple[Tensor, GenerationState]:
        """Append one token and return the next greedy token without logits."""
        return self.decode_step(input_ids, state, _next_token_only=True)

    def parameter_counts(self) -> dict[str, int]:
        total = sum(p.numel() for p in self.parameters())
        cfg = self.config
        inactive = cfg.n_layers * (cfg.n_experts - cfg.top_k) * 3 * cfg.dim * cfg.expert_dim
        return {"total": total, "active_per_token": total - inactive}
