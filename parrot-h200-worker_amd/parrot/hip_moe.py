"""PyTorch-ROCm host side of the MI355X inference MoE path.

Drop-in counterpart of the reference's Metal bridge (parrot/metal_moe.py):
the same operator contract -- route, grouped experts, RMSNorm, depth mix and
depth mix + RMSNorm -- backed by the gfx950 HIP kernels in
``parrot/kernels/*.hip`` through the C ABI of ``include/parrot_hip.h``.

Every function runs on PyTorch's current HIP stream, allocates its outputs
and workspaces with torch on the input's device, never synchronises with the
host and never falls back to another backend: unsupported inputs raise.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import TYPE_CHECKING

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _abi
from ._abi import ptr

if TYPE_CHECKING:
    from .model import MoE

MAX_EXPERTS = 32
MAX_DEPTH_SOURCES = 9


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(x: Tensor, what: str, dtypes=(torch.bfloat16,)) -> None:
    """Preconditions shared by every HIP operator (cf. parrot/metal_moe.py:154-157)."""
    if x.device.type != "cuda":
        raise RuntimeError(f"{what} requires a ROCm (cuda) tensor, got {x.device}")
    if x.dtype not in dtypes:
        raise RuntimeError(f"{what} requires {', '.join(map(str, dtypes))}, got {x.dtype}")
    if torch.is_grad_enabled():
        raise RuntimeError(f"{what} is inference-only; disable gradients")


def _capturing() -> bool:
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _scratch(owner, name: str, nbytes: int, device: torch.device) -> Tensor:
    """Reusable byte workspace kept outside the module's state_dict
    (cf. parrot/metal_moe.py:15-23), grown to the next power of two.

    An outgrown buffer is dropped, unless a HIP graph capture used it: the
    captured graph reads and writes it on every replay, so it stays
    referenced (in ``_hip_captured_scratch``) for as long as the owner
    lives.  Retention is therefore bounded by the captures, not by the
    sizes seen."""
    cached = owner.__dict__.get(name)
    if cached is None or cached.numel() < nbytes or cached.device != device:
        if cached is not None and owner.__dict__.get(name + "_captured", False):
            owner.__dict__.setdefault("_hip_captured_scratch", []).append(cached)
        size = 256
        while size < nbytes:
            size *= 2
        cached = torch.empty(size, dtype=torch.uint8, device=device)
        owner.__dict__[name] = cached
        owner.__dict__[name + "_captured"] = False
    if _capturing():
        owner.__dict__[name + "_captured"] = True
    return cached


def capacity(tokens: int, experts: int) -> int:
    """C = max(8, roundup8(ceil(2 * assignments / E))) (parrot/metal_moe.py:388-391)."""
    assignments = 2 * tokens
    return max(8, ((2 * assignments + experts - 1) // experts + 7) // 8 * 8)


@dataclass
class Grouping:
    """Deterministic expert grouping of the 2T assignments a = 2t + k.

    positions[a]: stable slot of a among its expert's assignments;
    counts[e]; offsets[: E + 1] exclusive prefix of counts and
    offsets[E + 1 :] of max(0, counts - C); perm[e, s] = assignment in
    slot s < C (-1 if empty); overflow[: offsets[2E + 1]] = assignments with
    slot >= C, expert-contiguous, ascending a within an expert.
    """
    positions: Tensor
    counts: Tensor
    offsets: Tensor
    perm: Tensor
    overflow: Tensor
    capacity: int

    @property
    def overflow_count(self) -> Tensor:
        return self.offsets[-1]


@dataclass
class RouteResult:
    probabilities: Tensor | None
    weights: Tensor
    indices: Tensor
    grouping: Grouping | None
    logits: Tensor | None = None
    # The route block table (route_top2(..., blocks=True)): uint8
    # [ceil(T / 16), 64], what the gate/up launch groups from past the sizes
    # it groups from the indices.
    blocks: Tensor | None = None

    def __iter__(self):
        """Unpacks as metal_route's 5-tuple (parrot/metal_moe.py:58-81):
        ``probabilities, weights, indices, positions, counts =
        hip_moe.route(module, flat, collect_stats)``, the call site of
        parrot/model.py:515-519.  Without a grouping (route_top2) positions
        and counts are None."""
        g = self.grouping
        return iter((self.probabilities, self.weights, self.indices,
                     None if g is None else g.positions, None if g is None else g.counts))


def _alloc_grouping(tokens: int, experts: int, cap: int, device) -> Grouping:
    i32 = dict(dtype=torch.int32, device=device)
    return Grouping(
        positions=torch.empty(2 * tokens, **i32),
        counts=torch.empty(experts, **i32),
        offsets=torch.empty(2 * experts + 2, **i32),
        perm=torch.empty((experts, cap), **i32),
        overflow=torch.empty(max(2 * tokens, 1), **i32),
        capacity=cap,
    )


def _route_workspace(owner, tokens: int, experts: int, device) -> tuple[Tensor, int]:
    nbytes = _abi.load().parrot_route_workspace_bytes(tokens, experts)
    return _scratch(owner, "_hip_route_workspace", nbytes, device), nbytes


# ---------------------------------------------------------------------------
# routing (cf. metal_route, parrot/metal_moe.py:58-81)
# ---------------------------------------------------------------------------

def route(module: "MoE", flat: Tensor, collect_stats: bool,
          logit_bias: Tensor | None = None, return_logits: bool = False) -> RouteResult:
    """Router projection + softmax top-2 + deterministic grouping."""
    _require(flat, "HIP routing")
    tokens, dim = flat.shape
    experts = module.cfg.n_experts
    if experts > MAX_EXPERTS or module.cfg.top_k != 2:
        raise RuntimeError(f"HIP routing supports top-2 of at most {MAX_EXPERTS} experts")
    flat = flat.contiguous()
    router_w = module.router.weight
    if router_w.dtype != flat.dtype or not router_w.is_contiguous():
        raise RuntimeError("router weight must be contiguous and match the input dtype")
    dev = flat.device
    cap = capacity(tokens, experts)
    f32 = dict(dtype=torch.float32, device=dev)
    probs = torch.empty((tokens, experts), **f32) if collect_stats else None
    logits = torch.empty((tokens, experts), **f32) if return_logits else None
    weights = torch.empty((tokens, 2), **f32)
    indices = torch.empty((tokens, 2), dtype=torch.int64, device=dev)
    g = _alloc_grouping(tokens, experts, cap, dev)
    if logit_bias is not None:
        logit_bias = logit_bias.to(device=dev, dtype=torch.float32).contiguous()
    ws, nbytes = _route_workspace(module, tokens, experts, dev)
    lib = _abi.load()
    _abi.check(lib.parrot_route_bf16(
        ptr(flat), ptr(router_w), ptr(logit_bias), tokens, dim, experts, cap,
        ptr(logits), ptr(probs), ptr(weights), ptr(indices), ptr(g.positions), ptr(g.counts),
        ptr(g.offsets), ptr(g.perm), ptr(g.overflow), ptr(ws), nbytes, _stream(dev)),
        "parrot_route_bf16")
    module.__dict__["_hip_grouping"] = g
    return RouteResult(probs, weights, indices, g, logits)


def route_top2(module: "MoE", flat: Tensor, logit_bias: Tensor | None = None,
               blocks: bool = False) -> RouteResult:
    """The router and top-2 of ``route`` alone (the same weights and indices
    to the bit), without grouping: for expert launches that group the
    indices themselves (``group_mode``).  ``blocks``: also the route block
    table (per 16 tokens: their 32 expert ids and the count per expert),
    which those launches group from past 2048 assignments."""
    _require(flat, "HIP routing")
    tokens, dim = flat.shape
    experts = module.cfg.n_experts
    if experts > MAX_EXPERTS or module.cfg.top_k != 2:
        raise RuntimeError(f"HIP routing supports top-2 of at most {MAX_EXPERTS} experts")
    flat = flat.contiguous()
    router_w = module.router.weight
    if router_w.dtype != flat.dtype or not router_w.is_contiguous():
        raise RuntimeError("router weight must be contiguous and match the input dtype")
    dev = flat.device
    weights = torch.empty((tokens, 2), dtype=torch.float32, device=dev)
    indices = torch.empty((tokens, 2), dtype=torch.int64, device=dev)
    if logit_bias is not None:
        logit_bias = logit_bias.to(device=dev, dtype=torch.float32).contiguous()
    if blocks:
        table = torch.empty(((tokens + 15) // 16, 64), dtype=torch.uint8, device=dev)
        _abi.check(_abi.load().parrot_route_top2_blocks_bf16(
            ptr(flat), ptr(router_w), ptr(logit_bias), tokens, dim, experts, ptr(weights),
            ptr(indices), ptr(table), _stream(dev)), "parrot_route_top2_blocks_bf16")
        return RouteResult(None, weights, indices, None, blocks=table)
    _abi.check(_abi.load().parrot_route_top2_bf16(
        ptr(flat), ptr(router_w), ptr(logit_bias), tokens, dim, experts, ptr(weights),
        ptr(indices), _stream(dev)), "parrot_route_top2_bf16")
    return RouteResult(None, weights, indices, None)


def route_for_experts(module: "MoE", flat: Tensor) -> RouteResult:
    """The routing an inference MoE layer needs before its expert launches:
    top-2 only where the gate/up launch groups the indices itself (with the
    route block table where it groups from that), else the top-2 with its
    grouping."""
    mode = group_mode(module, flat.shape[0], flat.shape[1])
    if mode == GROUP_FROM_IDS:
        return route_top2(module, flat)
    if mode == GROUP_FROM_BLOCKS:
        return route_top2(module, flat, blocks=True)
    return route(module, flat, collect_stats=False)


def route_from_logits(logits: Tensor, logit_bias: Tensor | None = None,
                      collect_stats: bool = False) -> RouteResult:
    """Top-2 + grouping from given fp32 router logits [T, E] (parity entry)."""
    if logits.device.type != "cuda" or logits.dtype != torch.float32 or logits.ndim != 2:
        raise RuntimeError("route_from_logits requires fp32 [tokens, experts] ROCm logits")
    tokens, experts = logits.shape
    logits = logits.contiguous()
    dev = logits.device
    cap = capacity(tokens, experts)
    f32 = dict(dtype=torch.float32, device=dev)
    probs = torch.empty((tokens, experts), **f32) if collect_stats else None
    weights = torch.empty((tokens, 2), **f32)
    indices = torch.empty((tokens, 2), dtype=torch.int64, device=dev)
    g = _alloc_grouping(tokens, experts, cap, dev)
    if logit_bias is not None:
        logit_bias = logit_bias.to(device=dev, dtype=torch.float32).contiguous()
    lib = _abi.load()
    nbytes = lib.parrot_route_workspace_bytes(tokens, experts)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
    _abi.check(lib.parrot_route_from_logits_f32(
        ptr(logits), ptr(logit_bias), tokens, experts, cap, ptr(probs), ptr(weights),
        ptr(indices), ptr(g.positions), ptr(g.counts), ptr(g.offsets), ptr(g.perm),
        ptr(g.overflow), ptr(ws), nbytes, _stream(dev)), "parrot_route_from_logits_f32")
    return RouteResult(probs, weights, indices, g)


def group_indices(indices: Tensor, experts: int, cap: int | None = None) -> Grouping:
    """Deterministic grouping of caller-supplied top-2 indices
    (cf. moe_count_assignments, parrot/kernels/moe_bf16.metal:650-660)."""
    if indices.device.type != "cuda" or indices.dtype != torch.int64 or indices.shape[-1] != 2:
        raise RuntimeError("group_indices requires int64 [tokens, 2] ROCm indices")
    indices = indices.reshape(-1, 2).contiguous()
    tokens = indices.shape[0]
    dev = indices.device
    cap = capacity(tokens, experts) if cap is None else cap
    g = _alloc_grouping(tokens, experts, cap, dev)
    lib = _abi.load()
    nbytes = lib.parrot_route_workspace_bytes(tokens, experts)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
    _abi.check(lib.parrot_group_indices(
        ptr(indices), tokens, experts, cap, ptr(g.positions), ptr(g.counts), ptr(g.offsets),
        ptr(g.perm), ptr(g.overflow), ptr(ws), nbytes, _stream(dev)), "parrot_group_indices")
    return g


# ---------------------------------------------------------------------------
# packed expert weights (cf. pack_combined_weights, parrot/metal_moe.py:105-131)
# ---------------------------------------------------------------------------

def _interleave_gate_up(gate: Tensor, up: Tensor) -> Tensor:
    """[..., H, dim] x 2 -> [..., 2H, dim] alternating 16 gate and 16 up rows."""
    *lead, hidden, dim = gate.shape
    g = gate.reshape(*lead, hidden // 16, 16, dim)
    u = up.reshape(*lead, hidden // 16, 16, dim)
    return torch.stack((g, u), dim=-3).reshape(*lead, 2 * hidden, dim)


def _fragment_order(w: Tensor) -> Tensor:
    """[..., N, K] row-major -> MFMA fragment order, same shape and size.

    Blocks of 16 rows x 32 k (1 KB) are laid out row-group-major, k-step
    minor; inside a block, lane l = 16 g + r of a wavefront holds row r,
    k = 8 g .. 8 g + 7 at bytes 16 l .. 16 l + 15 -- the operand layout of
    v_mfma_f32_16x16x32_bf16, so one wavefront load is 1 KB contiguous."""
    *lead, n, k = w.shape
    nd = len(lead)
    v = w.reshape(*lead, n // 16, 16, k // 32, 4, 8)
    order = list(range(nd)) + [nd, nd + 2, nd + 3, nd + 1, nd + 4]
    return v.permute(*order).contiguous().reshape(*lead, n, k)


def _expert_parameters(module: "MoE") -> list[Tensor]:
    params = [p for expert in module.experts
              for p in (expert.gate.weight, expert.up.weight, expert.down.weight)]
    return params + [module.shared.gate.weight, module.shared.up.weight,
                     module.shared.down.weight]


def pack_expert_weights(module: "MoE") -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(gate_up [E, 2H, dim], down [E, dim, H], shared_gate_up [2Hs, dim],
    shared_down [dim, Hs]) in MFMA fragment order (``_fragment_order``), the
    gate/up matrices with 16 gate rows then 16 up rows per 32-row group;
    cached until a parameter changes.  As in the reference, an eval-mode
    module under no-grad reuses the cache without re-checking versions; call
    ``invalidate_packed_weights`` after editing weights in place in that mode."""
    cached = module.__dict__.get("_hip_packed")
    if cached is not None and not torch.is_grad_enabled() and not module.training:
        return cached[1]
    params = _expert_parameters(module)
    version = tuple((p._version, p.device, p.dtype, p.data_ptr()) for p in params)
    if cached is not None and cached[0] == version:
        return cached[1]
    with torch.no_grad():
        gate = torch.stack([e.gate.weight.detach() for e in module.experts])
        up = torch.stack([e.up.weight.detach() for e in module.experts])
        packed = (
            _fragment_order(_interleave_gate_up(gate, up)),
            _fragment_order(torch.stack([e.down.weight.detach() for e in module.experts])),
            _fragment_order(_interleave_gate_up(module.shared.gate.weight.detach(),
                                                module.shared.up.weight.detach())),
            _fragment_order(module.shared.down.weight.detach()),
        )
    module.__dict__["_hip_packed"] = (version, packed)
    return packed


_PACKED_CACHES = ("_hip_packed", "_qkv_weight", "_absorbed_weights", "_absorbed_f32_weights")


def invalidate_packed_weights(module: torch.nn.Module) -> None:
    """Drop every packed / derived weight cached on ``module`` and its
    submodules (expert packs, packed projections, absorbed MLA maps)."""
    for sub in module.modules():
        for key in [k for k in sub.__dict__
                    if k in _PACKED_CACHES or k.startswith("_packed_linear_")]:
            del sub.__dict__[key]


# ---------------------------------------------------------------------------
# grouped experts (cf. grouped_mps_experts, parrot/metal_moe.py:372-416)
# ---------------------------------------------------------------------------

def grouped_hip_experts(module: "MoE", flat: Tensor, indices: Tensor, weights: Tensor,
                        positions: Tensor | None = None, counts: Tensor | None = None,
                        addend: Tensor | None = None, grouping: Grouping | None = None,
                        then_mix: tuple | None = None, route_blocks: Tensor | None = None):
    """Routed + shared SwiGLU experts and weighted combine; returns
    ``addend + delta`` (each rounded to the input dtype) when ``addend`` is
    given, else the MoE delta.

    ``then_mix = (depth_module, sources, output_norm)``: the combine also runs
    the next module's depth mix over ``sources + [result]`` (the kernel's
    result row is the last source) and returns ``(result, normalised mix)``;
    ``sources`` are [tokens, dim] views in stream order.

    ``route_blocks``: the route block table of these indices
    (``route_top2(..., blocks=True)``), for the gate/up launch to group
    from where it cannot group from the indices."""
    _require(flat, "The grouped HIP backend")
    cfg = module.cfg
    tokens, dim = flat.shape
    experts = cfg.n_experts
    if cfg.top_k != 2 or experts > MAX_EXPERTS:
        raise RuntimeError(f"grouped HIP experts support top-2 of at most {MAX_EXPERTS} experts")
    flat = flat.contiguous()
    self_group = False
    if grouping is None:
        cached = module.__dict__.get("_hip_grouping")
        if positions is not None and cached is not None and cached.positions is positions:
            grouping = cached
        elif groups_in_kernel(module, tokens, dim):
            # The gate/up launch groups the indices itself.
            self_group = True
            route_blocks = None
        elif (route_blocks is not None and
              group_mode(module, tokens, dim) == GROUP_FROM_BLOCKS):
            # ... from the route block table.
            if route_blocks.dtype != torch.uint8 or route_blocks.shape != ((tokens + 15) // 16, 64):
                raise RuntimeError("route block table must be uint8 [ceil(tokens / 16), 64]")
            self_group = True
        else:
            # Slots are recomputed from the indices in the deterministic stable
            # order; the expert outputs do not depend on the slot order.
            grouping = group_indices(indices, experts)
    gate_up, down, shared_gate_up, shared_down = pack_expert_weights(module)
    if gate_up.dtype != flat.dtype:
        raise RuntimeError("expert weights must match the input dtype")
    if addend is not None:
        _require(addend, "MoE addend")
        addend = addend.reshape(tokens, dim).contiguous()
    weights = weights.to(torch.float32).contiguous()
    lib = _abi.load()
    nbytes = lib.parrot_experts_workspace_bytes(tokens, dim, cfg.expert_dim,
                                                cfg.shared_expert_dim)
    ws = _scratch(module, "_hip_experts_workspace", nbytes, flat.device)
    out = torch.empty_like(flat)
    stream = _stream(flat.device)
    if then_mix is None and not self_group:
        _abi.check(lib.parrot_grouped_experts_bf16(
            ptr(flat), tokens, dim, experts, cfg.expert_dim, cfg.shared_expert_dim,
            grouping.capacity, ptr(grouping.counts), ptr(grouping.offsets), ptr(grouping.perm),
            ptr(grouping.overflow), ptr(weights), ptr(gate_up), ptr(down), ptr(shared_gate_up),
            ptr(shared_down), ptr(addend), ptr(out), ptr(ws), nbytes, stream),
            "parrot_grouped_experts_bf16")
        return out
    if self_group:
        if indices.dtype != torch.int64 or indices.numel() != 2 * tokens:
            raise RuntimeError("top-2 indices must be int64 [tokens, 2]")
        indices = indices.reshape(-1).contiguous()
        cap = capacity(tokens, experts)
        n = experts + (2 * experts + 2) + 2 * tokens
        buf = _scratch(module, "_hip_group_buffers", 4 * n, flat.device)[:4 * n].view(torch.int32)
        counts, offsets = buf[:experts], buf[experts:3 * experts + 2]
        sorted_ids = buf[3 * experts + 2:]
        shape = (experts, cfg.expert_dim, cfg.shared_expert_dim, cap)
        if route_blocks is not None:
            _abi.check(lib.parrot_experts_gate_up_grouping_blocks_bf16(
                ptr(flat), tokens, dim, *shape, ptr(route_blocks.contiguous()), ptr(counts),
                ptr(offsets), ptr(sorted_ids), ptr(gate_up), ptr(shared_gate_up), ptr(ws),
                nbytes, stream), "parrot_experts_gate_up_grouping_blocks_bf16")
        else:
            _abi.check(lib.parrot_experts_gate_up_grouping_bf16(
                ptr(flat), tokens, dim, *shape, ptr(indices), ptr(counts), ptr(offsets),
                ptr(sorted_ids), ptr(gate_up), ptr(shared_gate_up), ptr(ws), nbytes, stream),
                "parrot_experts_gate_up_grouping_bf16")
        _abi.check(lib.parrot_experts_down_sorted_bf16(
            tokens, dim, *shape, ptr(counts), ptr(offsets), ptr(sorted_ids), ptr(weights),
            ptr(down), ptr(shared_down), ptr(ws), nbytes, stream),
            "parrot_experts_down_sorted_bf16")
    else:
        group_args = (experts, cfg.expert_dim, cfg.shared_expert_dim, grouping.capacity,
                      ptr(grouping.counts), ptr(grouping.offsets), ptr(grouping.perm),
                      ptr(grouping.overflow))
        _abi.check(lib.parrot_experts_gate_up_bf16(
            ptr(flat), tokens, dim, *group_args, ptr(gate_up), ptr(shared_gate_up), ptr(ws),
            nbytes, stream), "parrot_experts_gate_up_bf16")
        _abi.check(lib.parrot_experts_down_bf16(
            tokens, dim, *group_args, ptr(weights), ptr(down), ptr(shared_down), ptr(ws), nbytes,
            stream), "parrot_experts_down_bf16")
    if then_mix is None:
        _abi.check(lib.parrot_experts_combine_bf16(
            tokens, dim, cfg.expert_dim, cfg.shared_expert_dim, ptr(addend), ptr(out), ptr(ws),
            nbytes, stream), "parrot_experts_combine_bf16")
        return out
    depth, sources, output_norm = then_mix
    if len(sources) + 1 > MAX_DEPTH_SOURCES:
        raise RuntimeError(f"HIP depth mixing supports one to {MAX_DEPTH_SOURCES} sources")
    rows = []
    for src in sources:
        if src.shape[-1] != dim or src.numel() != flat.numel() or src.dtype != flat.dtype:
            raise RuntimeError("depth sources must match the MoE input")
        rows.append(src.reshape(tokens, dim).contiguous())
    array = _SourceArray(*([t.data_ptr() for t in rows] +
                           [out.data_ptr()] * (MAX_DEPTH_SOURCES - len(rows))))
    mixed = torch.empty_like(flat)
    _abi.check(lib.parrot_experts_combine_depth_mix_bf16(
        tokens, dim, cfg.expert_dim, cfg.shared_expert_dim, ptr(addend), ptr(out), ptr(ws),
        nbytes, ctypes.cast(array, ctypes.c_void_p), len(rows) + 1, ptr(depth.query),
        ptr(depth.norm.weight), float(depth.norm.eps), ptr(output_norm.weight),
        float(output_norm.eps), None, ptr(mixed), stream), "parrot_experts_combine_depth_mix_bf16")
    del rows
    return out, mixed


GROUP_NONE, GROUP_FROM_IDS, GROUP_FROM_BLOCKS = 0, 1, 2


def group_mode(module: "MoE", tokens: int, dim: int) -> int:
    """How the gate/up launch can group at this size, with no separate
    grouping pass (parrot_experts_group_in_kernel): GROUP_FROM_IDS from the
    top-2 indices, GROUP_FROM_BLOCKS from the route block table only, or
    GROUP_NONE."""
    cfg = module.cfg
    return int(_abi.load().parrot_experts_group_in_kernel(
        tokens, dim, cfg.n_experts, cfg.expert_dim, cfg.shared_expert_dim))


def groups_in_kernel(module: "MoE", tokens: int, dim: int) -> bool:
    """Whether the gate/up launch groups the top-2 indices themselves at
    this size (the form the routed depth mix feeds)."""
    return group_mode(module, tokens, dim) == GROUP_FROM_IDS


DECODE_MAX_TOKENS = 16  # rows the fused decode MoE takes


def decode_experts(module: "MoE", flat: Tensor | None, addend: Tensor | None = None,
                   logit_bias: Tensor | None = None, mix: tuple | None = None,
                   pending: tuple | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """The whole MoE layer for at most DECODE_MAX_TOKENS rows in two launches
    (route + gate/up + SwiGLU, then down + weighted combine): returns
    ``(out, indices [T, 2] int64, weights [T, 2] fp32)`` with ``out`` =
    ``addend + delta`` when an addend is given (cf. metal_experts_decode,
    parrot/metal_moe.py:182-221).  ``mix = (depth_module, sources, norm)``:
    the input rows are ``depth_mix_norm(depth_module, sources, norm)``, made
    inside the same launches (``flat`` is then None; dim <= 1024).
    ``pending = (contributions [T, lanes, dim] fp32, base [T, 1, dim] or
    None, resolved [T, 1, dim])`` with ``mix``: the last depth source is a
    deferred module output (the reference's PendingResidual), resolved in
    the launch as bf16(base + bf16(sum of the lanes)) into ``resolved``, as
    metal_depth_mix_norm_pending does (parrot/metal_moe.py:480-500); the
    sources' last entry is only a placeholder and ``addend`` may be
    ``resolved``."""
    cfg = module.cfg
    keep = None
    if pending is not None and mix is None:
        raise RuntimeError("a pending depth source needs the input mix in the launch")
    if mix is not None:
        mix_args, flat, keep = _decode_mix_args(mix)  # flat: shape, dtype, device of the rows
    _require(flat, "The fused HIP decode MoE")
    tokens, dim = flat.shape
    if tokens > DECODE_MAX_TOKENS:
        raise RuntimeError(f"the fused decode MoE takes at most {DECODE_MAX_TOKENS} rows")
    if cfg.top_k != 2 or cfg.n_experts > MAX_EXPERTS:
        raise RuntimeError(f"HIP experts support top-2 of at most {MAX_EXPERTS} experts")
    flat = flat.contiguous()
    gate_up, down, shared_gate_up, shared_down = pack_expert_weights(module)
    if addend is not None:
        _require(addend, "MoE addend")
        addend = addend.reshape(tokens, dim).contiguous()
    bias = None
    if logit_bias is not None:
        bias = logit_bias.to(device=flat.device, dtype=torch.float32).contiguous()
    lib = _abi.load()
    nbytes = lib.parrot_decode_moe_workspace_bytes(DECODE_MAX_TOKENS, cfg.expert_dim,
                                                   cfg.shared_expert_dim)
    ws = _scratch(module, "_hip_decode_workspace", nbytes, flat.device)
    out = torch.empty_like(flat)
    indices = torch.empty((tokens, 2), dtype=torch.int64, device=flat.device)
    weights = torch.empty((tokens, 2), dtype=torch.float32, device=flat.device)
    tail = (ptr(module.router.weight), ptr(bias), ptr(gate_up), ptr(down), ptr(shared_gate_up),
            ptr(shared_down), ptr(addend), ptr(out), ptr(indices), ptr(weights), ptr(ws), nbytes,
            _stream(flat.device))
    if mix is None:
        _abi.check(lib.parrot_decode_moe_bf16(
            ptr(flat), tokens, dim, cfg.n_experts, cfg.expert_dim, cfg.shared_expert_dim, *tail),
            "parrot_decode_moe_bf16")
        return out, indices, weights
    if pending is None:
        _abi.check(lib.parrot_depth_mix_decode_moe_bf16(
            *mix_args, tokens, dim, cfg.n_experts, cfg.expert_dim, cfg.shared_expert_dim, *tail),
            "parrot_depth_mix_decode_moe_bf16")
    else:
        contributions, base, resolved = pending
        if (contributions.dtype != torch.float32 or contributions.dim() != 3 or
                contributions.shape[0] != tokens or contributions.shape[2] != dim or
                not contributions.is_contiguous() or contributions.device != flat.device):
            raise RuntimeError("pending contributions must be contiguous fp32 [T, lanes, dim]")
        for t in (base, resolved):
            if t is not None and (t.dtype != flat.dtype or t.numel() != tokens * dim or
                                  not t.is_contiguous() or t.device != flat.device):
                raise RuntimeError("pending base / resolved rows must be contiguous [T, 1, dim]"
                                   " in the input dtype")
        _abi.check(lib.parrot_depth_mix_decode_moe_pending_bf16(
            *mix_args, ptr(contributions), contributions.shape[1], ptr(base), ptr(resolved),
            tokens, dim, cfg.n_experts, cfg.expert_dim, cfg.shared_expert_dim, *tail),
            "parrot_depth_mix_decode_moe_pending_bf16")
    del keep  # alive until the launch is enqueued (it is)
    return out, indices, weights


def vocab_logits(h: Tensor, weight: Tensor) -> Tensor:
    """fp32 logits ``h @ weight^T`` for bf16 rows h [..., dim] and the tied
    head weight [vocab, dim] (cf. the head F.linear, parrot/model.py:714-715):
    the products of the bf16 operands accumulate in fp32 and the result is
    written in fp32 (one library GEMM with an fp32 output type)."""
    _require(h, "HIP vocabulary head")
    if weight.dtype != h.dtype or weight.ndim != 2 or weight.shape[1] != h.shape[-1]:
        raise RuntimeError("head weight must be a [vocab, dim] tensor of h's dtype")
    flat = h.reshape(-1, h.shape[-1])
    out = torch.mm(flat, weight.t(), out_dtype=torch.float32)
    return out.view(*h.shape[:-1], weight.shape[0])


def vocab_argmax(h: Tensor, weight: Tensor, advance: Tensor | None = None,
                 out: Tensor | None = None) -> Tensor:
    """Greedy tokens argmax(h @ weight^T) over fp32 logits for h [..., dim]
    (at most 16 rows) and the head weight [vocab, dim]; returns int64 ids of
    shape h.shape[:-1] (cf. vocab_argmax_partials/reduce_bf16,
    parrot/kernels/moe_bf16.metal:1541-1621).  ``advance``: an int32 device
    counter the same launch increments by one (a decode step's position).
    ``out``: a contiguous int64 tensor of one id per row to write them into
    (a decode graph's input ids, so the next replay reads them in place)."""
    if advance is not None and (advance.dtype != torch.int32 or advance.device != h.device):
        raise RuntimeError("advance must be an int32 tensor on h's device")
    if out is not None and (out.dtype != torch.int64 or out.device != h.device or
                            not out.is_contiguous() or out.numel() != h.numel() // h.shape[-1]):
        raise RuntimeError("out must be a contiguous int64 tensor of one id per row on h's device")
    _require(h, "HIP vocabulary argmax")
    flat = h.reshape(-1, h.shape[-1]).contiguous()
    rows, dim = flat.shape
    vocab = weight.shape[0]
    if weight.dtype != h.dtype or weight.shape[1] != dim or not weight.is_contiguous():
        raise RuntimeError("head weight must be a contiguous [vocab, dim] tensor of h's dtype")
    lib = _abi.load()
    nbytes = lib.parrot_vocab_argmax_workspace_bytes(16, vocab)
    ws = _scratch(weight, "_hip_vocab_workspace", nbytes, h.device)
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=h.device)
    _abi.check(lib.parrot_vocab_argmax_bf16(ptr(flat), rows, dim, ptr(weight), vocab, ptr(out),
                                            ptr(advance), ptr(ws), nbytes, _stream(h.device)),
               "parrot_vocab_argmax_bf16")
    return out.view(h.shape[:-1])


# ---------------------------------------------------------------------------
# RoPE for the local attention layers
# ---------------------------------------------------------------------------

def rope_qkv(qkv: Tensor, cos: Tensor, sin: Tensor, heads: int, kv_heads: int, head_dim: int,
             start: int, expand_kv: bool, start_device: Tensor | None = None,
             vt_keys: int = 0) -> tuple[Tensor, Tensor, Tensor]:
    """Split a packed q|k|v projection [b, t, (H + 2 Hk) d] into head-major
    q [b, H, t, d], k, v [b, Hk or H, t, d] and rotate q and k by RoPE at
    positions start .. start + t - 1 (fp32 tables [max_positions, d / 2]),
    shifted by the device int32 ``start_device`` when given.  With
    ``vt_keys`` > 0 the values come back transposed, [b, Hk, d, vt_keys]
    (columns past t unwritten), the layout ``causal_attention`` reads."""
    _require(qkv, "HIP RoPE")
    b, t, width = qkv.shape
    if width != (heads + 2 * kv_heads) * head_dim:
        raise RuntimeError("packed q|k|v width does not match the head layout")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise RuntimeError("RoPE tables must be fp32")
    if start_device is not None and (start_device.dtype != torch.int32 or
                                     start_device.device != qkv.device):
        raise RuntimeError("start_device must be an int32 tensor on the projection's device")
    qkv = qkv.contiguous()
    kv_out = heads if expand_kv else kv_heads
    q = qkv.new_empty((b, heads, t, head_dim))
    k = qkv.new_empty((b, kv_out, t, head_dim))
    if vt_keys:
        v = qkv.new_empty((b, kv_heads, head_dim, vt_keys))
    else:
        v = qkv.new_empty((b, kv_out, t, head_dim))
    _abi.check(_abi.load().parrot_rope_qkv_bf16(
        ptr(qkv), ptr(cos), ptr(sin), b, t, start, ptr(start_device), cos.shape[0], heads,
        kv_heads, head_dim, int(expand_kv), vt_keys, ptr(q), ptr(k), ptr(v),
        _stream(qkv.device)), "parrot_rope_qkv_bf16")
    return q, k, v


# ---------------------------------------------------------------------------
# Dense projections of the attention layers (cf. parrot/model.py:167-230,
# 331-432; parrot/kernels/moe_bf16.metal:1364-1389 for the residual add)
# ---------------------------------------------------------------------------

def proj_supported(k: int, n: int) -> bool:
    """Shapes the projection kernels take: k % 64 == 0, k <= 2048, n % 16 == 0."""
    return 0 < k <= 2048 and k % 64 == 0 and n > 0 and n % 16 == 0


def pack_linear(owner, name: str, weights: tuple[Tensor, ...]) -> Tensor:
    """The row concatenation of ``weights`` ([n_i, k] each) in MFMA fragment
    order (``_fragment_order``), cached on ``owner`` (attribute
    ``_packed_linear_<name>``, so no method is shadowed) until a weight
    changes.  As for the expert weights, an eval-mode owner under no-grad
    reuses the cache without re-checking versions."""
    name = "_packed_linear_" + name
    cached = owner.__dict__.get(name)
    if cached is not None and not torch.is_grad_enabled() and not owner.training:
        return cached[1]
    version = tuple((p._version, p.device, p.dtype, p.data_ptr()) for p in weights)
    if cached is None or cached[0] != version:
        with torch.no_grad():
            w = torch.cat([p.detach() for p in weights], 0)
            cached = (version, _fragment_order(w.contiguous()))
        owner.__dict__[name] = cached
    return cached[1]


def _rows(x: Tensor) -> Tensor:
    """x as a [rows, k] matrix the projection kernels can read in place."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


def proj(x: Tensor, packed: Tensor, n: int, addend: Tensor | None = None) -> Tensor:
    """y = x W^T for x [..., k] and W [n, k] packed by ``pack_linear``; with
    ``addend`` [..., n], bf16(addend + bf16(x W^T)) (the residual add of the
    attention output)."""
    _require(x, "HIP projection")
    x2 = _rows(x)
    rows, k = x2.shape
    if packed.numel() != n * k:
        raise RuntimeError("packed projection weight does not match the input width")
    out = x.new_empty((*x.shape[:-1], n))
    add = None
    if addend is not None:
        if addend.shape != out.shape or addend.dtype != x.dtype:
            raise RuntimeError("projection addend must match the output")
        add = addend.reshape(rows, n).contiguous()
    _abi.check(_abi.load().parrot_proj_bf16(
        ptr(x2), rows, k, x2.stride(0), ptr(packed), n, ptr(add), n, ptr(out), n,
        _stream(x.device)), "parrot_proj_bf16")
    return out


def proj_transposed(x: Tensor, packed: Tensor, n: int, keys: int) -> Tensor:
    """(x W^T) transposed per sequence: x [b, t, k] -> [b, n, keys] with
    columns past t unwritten (``causal_attention``'s value layout)."""
    _require(x, "HIP projection")
    b, t, k = x.shape
    if packed.numel() != n * k:
        raise RuntimeError("packed projection weight does not match the input width")
    x = x.contiguous()
    out = x.new_empty((b, n, keys))
    _abi.check(_abi.load().parrot_proj_transposed_bf16(
        ptr(x), b, t, k, ptr(packed), n, keys, ptr(out), _stream(x.device)),
        "parrot_proj_transposed_bf16")
    return out


def proj_rope_qkv(x: Tensor, packed: Tensor, cos: Tensor, sin: Tensor, heads: int,
                  kv_heads: int, head_dim: int, start: int = 0,
                  start_device: Tensor | None = None,
                  vt_keys: int = 0) -> tuple[Tensor, Tensor, Tensor]:
    """The packed q|k|v projection of x [b, t, dim] fused with ``rope_qkv``
    (expand_kv off): the same q, k and v (or v transposed with ``vt_keys``),
    bit for bit, as ``rope_qkv(F.linear(x, W), ...)`` with W unpacked."""
    _require(x, "HIP projection")
    b, t, dim = x.shape
    n = (heads + 2 * kv_heads) * head_dim
    if packed.numel() != n * dim:
        raise RuntimeError("packed q|k|v weight does not match the head layout")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise RuntimeError("RoPE tables must be fp32")
    if start_device is not None and (start_device.dtype != torch.int32 or
                                     start_device.device != x.device):
        raise RuntimeError("start_device must be an int32 tensor on the input's device")
    x = x.contiguous()
    q = x.new_empty((b, heads, t, head_dim))
    k = x.new_empty((b, kv_heads, t, head_dim))
    v = x.new_empty((b, kv_heads, head_dim, vt_keys) if vt_keys else (b, kv_heads, t, head_dim))
    _abi.check(_abi.load().parrot_proj_rope_qkv_bf16(
        ptr(x), b, t, dim, ptr(packed), ptr(cos), ptr(sin), start, ptr(start_device),
        cos.shape[0], heads, kv_heads, head_dim, vt_keys, ptr(q), ptr(k), ptr(v),
        _stream(x.device)), "parrot_proj_rope_qkv_bf16")
    return q, k, v


def proj_rope_qkv_frag(x: Tensor, packed: Tensor, cos: Tensor, sin: Tensor, heads: int,
                       kv_heads: int, head_dim: int, cache_kv: bool = True):
    """``proj_rope_qkv`` writing K and V for ``causal_attention_frag``:
    returns (q [b, H, t, d], k_frag, v_frag, k, v) with row-major k, v
    [b, Hk, t, d] only when ``cache_kv`` (else None); k, v and the valid keys
    of k_frag, v_frag equal ``proj_rope_qkv``'s bit for bit."""
    _require(x, "HIP projection")
    b, t, dim = x.shape
    n = (heads + 2 * kv_heads) * head_dim
    if packed.numel() != n * dim:
        raise RuntimeError("packed q|k|v weight does not match the head layout")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise RuntimeError("RoPE tables must be fp32")
    x = x.contiguous()
    q = x.new_empty((b, heads, t, head_dim))
    frag = b * kv_heads * key_blocks(t) * 32 * head_dim
    kf = x.new_empty((b, kv_heads, frag // (b * kv_heads)))
    vf = torch.empty_like(kf)
    k = x.new_empty((b, kv_heads, t, head_dim)) if cache_kv else None
    v = x.new_empty((b, kv_heads, t, head_dim)) if cache_kv else None
    _abi.check(_abi.load().parrot_proj_rope_qkv_frag_bf16(
        ptr(x), b, t, dim, ptr(packed), ptr(cos), ptr(sin), 0, None, cos.shape[0], heads,
        kv_heads, head_dim, ptr(q), ptr(k), ptr(v), ptr(kf), ptr(vf), _stream(x.device)),
        "parrot_proj_rope_qkv_frag_bf16")
    return q, kf, vf, k, v


def proj_frag(x: Tensor, packed: Tensor, n: int, head_dim: int, values: bool) -> Tensor:
    """x [b, t, k] W^T stored as attention K (or V, ``values``) in fragment
    order for n / head_dim heads: [b, n / head_dim, ceil(t / 32) * 32 * d]."""
    _require(x, "HIP projection")
    b, t, k = x.shape
    if packed.numel() != n * k:
        raise RuntimeError("packed projection weight does not match the input width")
    x = x.contiguous()
    out = x.new_empty((b, n // head_dim, key_blocks(t) * 32 * head_dim))
    _abi.check(_abi.load().parrot_proj_frag_bf16(
        ptr(x), b, t, k, ptr(packed), n, head_dim, int(values), ptr(out), _stream(x.device)),
        "parrot_proj_frag_bf16")
    return out


def proj_kv_frag(x: Tensor, packed: Tensor, n: int, head_dim: int) -> tuple[Tensor, Tensor]:
    """Both MLA up-projections in one launch: ``packed`` holds [Wk; Wv]
    ([2n, k], ``pack_linear``), x [b, t, k] may be a row-strided view; returns
    (k_frag, v_frag) for n / head_dim heads, as two ``proj_frag`` calls would."""
    _require(x, "HIP projection")
    b, t, k = x.shape
    if packed.numel() != 2 * n * k:
        raise RuntimeError("packed [Wk; Wv] weight does not match the input width")
    x2 = _rows(x)
    kf = x.new_empty((b, n // head_dim, key_blocks(t) * 32 * head_dim))
    vf = torch.empty_like(kf)
    _abi.check(_abi.load().parrot_proj_kv_frag_bf16(
        ptr(x2), b, t, k, x2.stride(0), ptr(packed), n, head_dim, ptr(kf), ptr(vf),
        _stream(x.device)), "parrot_proj_kv_frag_bf16")
    return kf, vf


# ---------------------------------------------------------------------------
# Causal attention for prefill / forward (cf. parrot/model.py:264-295, 350-360)
# ---------------------------------------------------------------------------

ATTENTION_HEAD_DIMS = (64, 96, 128)


def padded_keys(t: int) -> int:
    """Key capacity of a transposed value tensor for ``causal_attention``."""
    return (t + 31) // 32 * 32


def causal_attention(q: Tensor, k: Tensor, v: Tensor | None = None, *, scale: float,
                     window: int | None = None, vt: Tensor | None = None) -> Tensor:
    """softmax(q k^T * scale) v with key j visible to query i iff
    i - window < j <= i, for q [b, H, t, d] and k [b, Hk, t, d] (any strides
    with a unit last stride; Hk divides H), and the values either as v
    [b, Hk, t, d] or already transposed as vt [b, Hk, d, >= padded_keys(t)]
    (unit stride along the keys).  Returns [b, t, H * d] bf16, the layout of
    the output projection's input."""
    _require(q, "HIP causal attention")
    b, heads, t, d = q.shape
    kv_heads = k.shape[1]
    if k.shape != (b, kv_heads, t, d) or heads % kv_heads:
        raise RuntimeError("attention shapes do not match")
    if d not in ATTENTION_HEAD_DIMS:
        raise RuntimeError(f"HIP attention supports head widths {ATTENTION_HEAD_DIMS}")
    if (v is None) == (vt is None):
        raise RuntimeError("pass exactly one of v and vt")
    if vt is None:
        if v.shape != k.shape:
            raise RuntimeError("attention shapes do not match")
        vt = v.new_empty((b, kv_heads, d, padded_keys(t)))
        vt[..., :t].copy_(v.transpose(-1, -2))
    elif vt.shape[:3] != (b, kv_heads, d) or vt.shape[3] < padded_keys(t):
        raise RuntimeError("transposed values must be [b, Hk, d, >= padded_keys(t)]")
    tensors = []
    for x in (q, k, vt):
        if x.stride(-1) != 1 or any(st % 8 for st in x.stride()[:3]) or x.data_ptr() % 16:
            x = x.contiguous()
        tensors.append(x)
    q, k, vt = tensors
    out = q.new_empty((b, t, heads * d))
    strides = [(ctypes.c_int64 * 3)(*x.stride()[:3]) for x in (q, k, vt)]
    _abi.check(_abi.load().parrot_causal_attention_bf16(
        ptr(q), ptr(k), ptr(vt), ctypes.cast(strides[0], ctypes.c_void_p),
        ctypes.cast(strides[1], ctypes.c_void_p), ctypes.cast(strides[2], ctypes.c_void_p),
        b, t, heads, kv_heads, d, t if window is None else window, scale, ptr(out),
        _stream(q.device)), "parrot_causal_attention_bf16")
    return out


# ---------------------------------------------------------------------------
# Decode-step attention over the generation caches (cf. parrot/model.py:239-262,
# 399-432; parrot/kernels/moe_bf16.metal:1203-1518)
# ---------------------------------------------------------------------------

def key_blocks(t: int) -> int:
    """Blocks of 32 keys in the fragment-order K / V of ``t`` positions."""
    return (t + 31) // 32


def pack_kv_fragments(k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
    """Row-major K, V [b, Hk, t, d] -> the fragment order that
    ``causal_attention_frag`` reads ([b, Hk, ceil(t / 32) * 32 * d] each):
    per block of 32 keys, K fragments (n, s) with lane 16 g + c holding key
    32 blk + 16 n + c, dims 32 s + 8 g .. + 7; V fragments t with lane
    16 g + c holding dim 16 t + c, keys 32 blk + {4 g .. + 3, 16 + 4 g .. + 3}.
    Padding keys are zero."""
    b, hk, t, d = k.shape
    nblk = key_blocks(t)
    pad = nblk * 32 - t
    kp = F.pad(k, (0, 0, 0, pad))
    vp = F.pad(v, (0, 0, 0, pad))
    kf = kp.reshape(b, hk, nblk, 2, 16, d // 32, 4, 8).permute(0, 1, 2, 3, 5, 6, 4, 7)
    vf = vp.reshape(b, hk, nblk, 2, 4, 4, d // 16, 16).permute(0, 1, 2, 6, 4, 7, 3, 5)
    return kf.contiguous().reshape(b, hk, -1), vf.contiguous().reshape(b, hk, -1)


def causal_attention_frag(q: Tensor, k_frag: Tensor, v_frag: Tensor, *, kv_heads: int,
                          scale: float, window: int | None = None) -> Tensor:
    """``causal_attention`` with K and V in fragment order (``pack_kv_fragments``
    or the fragment outputs of the projection kernels); q [b, H, t, d] with
    any strides that are multiples of 8.  Returns [b, t, H * d] bf16."""
    _require(q, "HIP causal attention")
    b, heads, t, d = q.shape
    if d not in ATTENTION_HEAD_DIMS:
        raise RuntimeError(f"head_dim {d} is not supported (64, 96, 128)")
    need = b * kv_heads * key_blocks(t) * 32 * d
    if k_frag.numel() != need or v_frag.numel() != need:
        raise RuntimeError("fragment-order K / V do not match the query shape")
    if q.stride(-1) != 1 or any(st % 8 for st in q.stride()[:3]) or q.data_ptr() % 16:
        q = q.contiguous()
    out = q.new_empty((b, t, heads * d))
    st = (ctypes.c_int64 * 3)(*q.stride()[:3])
    _abi.check(_abi.load().parrot_causal_attention_frag_bf16(
        ptr(q), ctypes.cast(st, ctypes.c_void_p), ptr(k_frag), ptr(v_frag), b, t, heads, kv_heads, d,
        t if window is None else window, scale, ptr(out), _stream(q.device)),
        "parrot_causal_attention_frag_bf16")
    return out


# Output widths and head count for which an attention output's projection
# can be deferred per head to the next depth mix (the kernels' instances).
ATTENTION_OUT_WIDTHS = (512, 768, 1024)
PENDING_HEADS = 8


def attention_heads_out_supported(heads: int, head_dim: int, dim: int) -> bool:
    """Whether causal_attention_frag_out takes these shapes and the depth
    mix can sum its contributions (parrot_depth_mix_route_pending_bf16)."""
    return (heads == PENDING_HEADS and head_dim in ATTENTION_HEAD_DIMS and
            dim in ATTENTION_OUT_WIDTHS and dim % 32 == 0)


def causal_attention_frag_out(q: Tensor, k_frag: Tensor, v_frag: Tensor, out_packed: Tensor,
                              dim: int, *, kv_heads: int, scale: float,
                              window: int | None = None) -> Tensor:
    """``causal_attention_frag`` with the output projection deferred per
    head: returns fp32 contributions [b, t, H, dim], head h's share
    bf16(y_h) W[:, h d : h d + d]^T of the projection by ``out_packed`` (the
    output weight packed by ``pack_linear``).  bf16 of their sum over heads
    is ``proj(y, out_packed, dim)`` up to fp32 summation order (cf. the
    reference's defer_sum, parrot/model.py:301-316)."""
    _require(q, "HIP causal attention")
    b, heads, t, d = q.shape
    if not attention_heads_out_supported(heads, d, dim):
        raise RuntimeError(f"no deferred output projection for {heads} heads of {d}, width {dim}")
    need = b * kv_heads * key_blocks(t) * 32 * d
    if k_frag.numel() != need or v_frag.numel() != need:
        raise RuntimeError("fragment-order K / V do not match the query shape")
    if out_packed.numel() != dim * heads * d:
        raise RuntimeError("packed output weight does not match [dim, heads * head_dim]")
    if q.stride(-1) != 1 or any(st % 8 for st in q.stride()[:3]) or q.data_ptr() % 16:
        q = q.contiguous()
    out = torch.empty((b, t, heads, dim), dtype=torch.float32, device=q.device)
    st = (ctypes.c_int64 * 3)(*q.stride()[:3])
    _abi.check(_abi.load().parrot_causal_attention_frag_out_bf16(
        ptr(q), ctypes.cast(st, ctypes.c_void_p), ptr(k_frag), ptr(v_frag), b, t, heads, kv_heads,
        d, t if window is None else window, scale, ptr(out_packed), dim, ptr(out),
        _stream(q.device)), "parrot_causal_attention_frag_out_bf16")
    return out


def _check_position(position: Tensor, device: torch.device) -> None:
    if position.dtype != torch.int32 or position.device != device or position.numel() != 1:
        raise RuntimeError("position must be a one-element int32 tensor on the cache's device")


def decode_attention(q: Tensor, k_new: Tensor, v_new: Tensor, key_cache: Tensor,
                     value_cache: Tensor, position: Tensor, window: int,
                     scale: float) -> Tensor:
    """One decode step of sliding-window GQA: store k_new / v_new [b, Hk, 1, d]
    at cache position p = position (device int32) and attend q [b, H, 1, d]
    over positions max(0, p - window + 1) .. p.  Returns [b, H * d] bf16."""
    _require(q, "HIP decode attention")
    b, heads, t, d = q.shape
    _, kv_heads, max_pos, _ = key_cache.shape
    if t != 1 or k_new.shape != (b, kv_heads, 1, d) or v_new.shape != k_new.shape:
        raise RuntimeError("decode attention takes one new position per sequence")
    if key_cache.shape != (b, kv_heads, max_pos, d) or value_cache.shape != key_cache.shape:
        raise RuntimeError("cache shapes do not match the heads")
    if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
        raise RuntimeError("caches must be contiguous")
    _check_position(position, q.device)
    q, k_new, v_new = q.contiguous(), k_new.contiguous(), v_new.contiguous()
    out = q.new_empty((b, heads * d))
    _abi.check(_abi.load().parrot_decode_attention_bf16(
        ptr(q), ptr(k_new), ptr(v_new), ptr(key_cache), ptr(value_cache), ptr(position),
        b, heads, kv_heads, d, max_pos, window, scale, ptr(out), _stream(q.device)),
        "parrot_decode_attention_bf16")
    return out


DEFER_MAX_TOKENS = 4  # rows up to which decode attention defers its output sum
DECODE_HEADS_PARTS = 16  # workgroups per head of parrot_decode_attention_heads_bf16


def decode_attention_heads_supported(tokens: int, dim: int, heads: int, kv_heads: int,
                                     head_dim: int, max_positions: int, window: int) -> bool:
    """Shapes for which a decode step defers the attention output sum
    (``decode_attention_heads`` + the pending decode MoE mix): at most
    DEFER_MAX_TOKENS rows, since each head's attention runs in
    DECODE_HEADS_PARTS workgroups (one per 1/16 of the output columns), and
    the shape limits both kernels check (parrot_decode_attention_heads_check:
    at most 16 heads, one pending lane each, and the heads kernel's LDS).
    Other shapes take the undeferred decode."""
    if not 1 <= tokens <= DEFER_MAX_TOKENS:
        return False
    return _abi.load().parrot_decode_attention_heads_check(
        tokens, heads, kv_heads, head_dim, max_positions, window, dim) == 0


def decode_attention_heads(q: Tensor, k_new: Tensor, v_new: Tensor, key_cache: Tensor,
                           value_cache: Tensor, position: Tensor, window: int, scale: float,
                           out_weight: Tensor) -> Tensor:
    """``decode_attention`` with the output projection deferred per head (the
    reference's defer_sum, parrot/model.py:301-316): returns contributions
    [b, H, dim] fp32, contributions[b, h] = y_bf16[b, h] @ out_weight[:, h d :
    h d + d]^T.  Their sum over heads, rounded to bf16 and added to the
    addend, is the attention module's output; ``decode_experts(...,
    pending=...)`` resolves it inside its input mix."""
    _require(q, "HIP decode attention")
    b, heads, t, d = q.shape
    _, kv_heads, max_pos, _ = key_cache.shape
    if t != 1 or k_new.shape != (b, kv_heads, 1, d) or v_new.shape != k_new.shape:
        raise RuntimeError("decode attention takes one new position per sequence")
    if key_cache.shape != (b, kv_heads, max_pos, d) or value_cache.shape != key_cache.shape:
        raise RuntimeError("cache shapes do not match the heads")
    if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
        raise RuntimeError("caches must be contiguous")
    dim = out_weight.shape[0]
    if (out_weight.dtype != q.dtype or out_weight.shape != (dim, heads * d) or
            not out_weight.is_contiguous()):
        raise RuntimeError("output projection must be a contiguous [dim, heads * head_dim] "
                           "weight of q's dtype")
    _check_position(position, q.device)
    q, k_new, v_new = q.contiguous(), k_new.contiguous(), v_new.contiguous()
    out = torch.empty((b, heads, dim), dtype=torch.float32, device=q.device)
    _abi.check(_abi.load().parrot_decode_attention_heads_bf16(
        ptr(q), ptr(k_new), ptr(v_new), ptr(key_cache), ptr(value_cache), ptr(position),
        b, heads, kv_heads, d, max_pos, window, scale, ptr(out_weight), dim, ptr(out),
        _stream(q.device)), "parrot_decode_attention_heads_bf16")
    return out


def decode_qkv_supported(tokens: int, dim: int, heads: int, kv_heads: int,
                         head_dim: int) -> bool:
    """Shapes parrot_decode_qkv_bf16 takes."""
    return (1 <= tokens <= 16 and dim % 128 == 0 and dim <= 1024 and head_dim % 2 == 0
            and (heads + 2 * kv_heads) * head_dim % 16 == 0)


def decode_qkv(x: Tensor | None, weight: Tensor, cos: Tensor, sin: Tensor, heads: int,
               kv_heads: int, head_dim: int, position: Tensor,
               mix: tuple | None = None,
               embed: tuple | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """A decode step's q|k|v projection + RoPE at the device ``position`` in
    one launch: x [b, 1, dim] bf16, or ``mix = (depth_module, sources, norm)``
    whose ``depth_mix_norm`` the launch computes itself; ``weight`` the
    stacked row-major q|k|v weight.  Returns q [b, heads, 1, d], k and v
    [b, kv_heads, 1, d] (cf. LocalGQA.decode, parrot/model.py:176-262).

    ``embed = (token_ids [b, 1] int64, embedding weight [vocab, dim])`` with a
    one-source ``mix``: the source is the tokens' embedding rows, gathered in
    the same launch and written into that source tensor (the reference's
    ``self.embedding(input_ids)``, parrot/model.py:830)."""
    if embed is not None:
        return _decode_qkv_embed(weight, cos, sin, heads, kv_heads, head_dim, position, mix,
                                 embed)
    keep = None
    if mix is not None:
        mix_args, ref, keep = _decode_mix_args(mix)
        mix_args = (None,) + mix_args
    else:
        ref = x.reshape(x.shape[0], x.shape[-1]).contiguous()
        mix_args = (ptr(ref), None, 0, None, None, 0.0, None, 0.0)
    _require(ref, "HIP decode q|k|v projection")
    b, dim = ref.shape
    if weight.dtype != ref.dtype or not weight.is_contiguous():
        raise RuntimeError("q|k|v weight must be contiguous in the input's dtype")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise RuntimeError("RoPE tables must be fp32")
    _check_position(position, ref.device)
    q = ref.new_empty((b, heads, 1, head_dim))
    k = ref.new_empty((b, kv_heads, 1, head_dim))
    v = ref.new_empty((b, kv_heads, 1, head_dim))
    _abi.check(_abi.load().parrot_decode_qkv_bf16(
        *mix_args, b, dim, ptr(weight), heads, kv_heads, head_dim, ptr(cos), ptr(sin),
        cos.shape[0], ptr(position), ptr(q), ptr(k), ptr(v), _stream(ref.device)),
        "parrot_decode_qkv_bf16")
    del keep  # alive until the launch is enqueued (it is)
    return q, k, v


def _decode_qkv_embed(weight: Tensor, cos: Tensor, sin: Tensor, heads: int, kv_heads: int,
                      head_dim: int, position: Tensor, mix: tuple,
                      embed: tuple) -> tuple[Tensor, Tensor, Tensor]:
    ids, table = embed
    depth, sources, norm = mix
    if len(sources) != 1:
        raise RuntimeError("the embedded q|k|v launch mixes exactly one source")
    out = sources[0]
    _require(out, "HIP decode q|k|v projection")
    b, dim = out.numel() // out.shape[-1], out.shape[-1]
    if not out.is_contiguous():
        raise RuntimeError("embedding output must be contiguous")
    if ids.dtype != torch.int64 or ids.numel() != b or ids.device != out.device:
        raise RuntimeError("token ids must be int64 [b, 1] on the output's device")
    if (table.dtype != out.dtype or table.dim() != 2 or table.shape[1] != dim or
            not table.is_contiguous()):
        raise RuntimeError("embedding table must be a contiguous [vocab, dim] weight of the "
                           "output dtype")
    if weight.dtype != out.dtype or not weight.is_contiguous():
        raise RuntimeError("q|k|v weight must be contiguous in the input's dtype")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise RuntimeError("RoPE tables must be fp32")
    _check_position(position, out.device)
    ids = ids.contiguous()
    q = out.new_empty((b, heads, 1, head_dim))
    k = out.new_empty((b, kv_heads, 1, head_dim))
    v = out.new_empty((b, kv_heads, 1, head_dim))
    _abi.check(_abi.load().parrot_decode_qkv_embed_bf16(
        ptr(ids), ptr(table), table.shape[0], ptr(out), ptr(depth.query),
        ptr(depth.norm.weight), float(depth.norm.eps), ptr(norm.weight), float(norm.eps), b, dim,
        ptr(weight), heads, kv_heads, head_dim, ptr(cos), ptr(sin), cos.shape[0], ptr(position),
        ptr(q), ptr(k), ptr(v), _stream(out.device)), "parrot_decode_qkv_embed_bf16")
    return q, k, v


MLA_DECODE_MAX_TOKENS = 16


def mla_decode_supported(tokens: int, dim: int, width: int) -> bool:
    """Shapes parrot_mla_decode_in/out_bf16 take (width = heads x latent)."""
    return (1 <= tokens <= MLA_DECODE_MAX_TOKENS and dim % 128 == 0 and dim <= 2048
            and width % 128 == 0 and width <= 2048 and tokens * width * 4 <= 65536)


def _decode_mix_args(mix: tuple) -> tuple[tuple, Tensor, list[Tensor]]:
    """C-ABI arguments (sources .. norm eps) of a decode launch that makes
    its input as ``depth_mix_norm(*mix)``; also the first source row block
    (shape, dtype and device of the input) and the rows to keep alive."""
    depth, sources, norm = mix
    first = sources[0]
    b, dim = first.numel() // first.shape[-1], first.shape[-1]
    rows = [s.reshape(b, dim).contiguous() for s in sources]
    for s in rows:
        if s.dtype != first.dtype or s.device != first.device:
            raise RuntimeError("depth sources must share shape, dtype and device")
    if not 1 <= len(rows) <= MAX_DEPTH_SOURCES:
        raise RuntimeError(f"HIP depth mixing supports one to {MAX_DEPTH_SOURCES} sources")
    array = _SourceArray(*([t.data_ptr() for t in rows] +
                           [rows[0].data_ptr()] * (MAX_DEPTH_SOURCES - len(rows))))
    args = (ctypes.cast(array, ctypes.c_void_p), len(rows), ptr(depth.query),
            ptr(depth.norm.weight), float(depth.norm.eps), ptr(norm.weight), float(norm.eps))
    return args, rows[0], rows + [array]


def mla_decode_in(x: Tensor | None, absorbed_query: Tensor, kv_down: Tensor,
                  mix: tuple | None = None) -> tuple[Tensor, Tensor]:
    """The MLA decode step's projections in one launch: x [b, 1, dim] bf16
    (or ``mix = (depth_module, sources, norm)``, whose ``depth_mix_norm`` the
    launch computes itself) -> (q_latent [b, H * r] fp32 = x.float()
    absorbed_query.float()^T, latent [b, 1, r] bf16 = kv_down(x)); cf.
    parrot/model.py:417-422."""
    keep = None
    if mix is not None:
        mix_args, ref, keep = _decode_mix_args(mix)
        mix_args = (None,) + mix_args
    else:
        ref = x.reshape(x.shape[0], x.shape[-1]).contiguous()
        mix_args = (ptr(ref), None, 0, None, None, 0.0, None, 0.0)
    _require(ref, "HIP MLA decode projections")
    b, dim = ref.shape
    for w in (absorbed_query, kv_down):
        if w.dtype != ref.dtype or not w.is_contiguous() or w.shape[-1] != dim:
            raise RuntimeError("MLA decode weights must be contiguous [rows, dim] in x's dtype")
    q = torch.empty((b, absorbed_query.shape[0]), dtype=torch.float32, device=ref.device)
    latent = torch.empty((b, 1, kv_down.shape[0]), dtype=ref.dtype, device=ref.device)
    _abi.check(_abi.load().parrot_mla_decode_in_bf16(
        *mix_args, b, dim, ptr(absorbed_query), absorbed_query.shape[0], ptr(kv_down),
        kv_down.shape[0], ptr(q), ptr(latent), _stream(ref.device)), "parrot_mla_decode_in_bf16")
    del keep  # alive until the launch is enqueued (it is)
    return q, latent


def decode_linear(x: Tensor, weight: Tensor, addend: Tensor | None = None) -> Tensor:
    """bf16(x weight^T) [.., n] (+ addend, a bf16 sum) for at most 16 rows
    in one launch; x [.., k] bf16, weight [n, k] (cf. the decode output
    projection of LocalGQA, parrot/model.py:167-230)."""
    _require(x, "HIP decode linear")
    k = x.shape[-1]
    rows = x.numel() // k
    n = weight.shape[0]
    if weight.dtype != x.dtype or not weight.is_contiguous() or weight.shape[1] != k:
        raise RuntimeError("decode linear weight must be contiguous [n, k] in x's dtype")
    x2 = x.reshape(rows, k).contiguous()
    out = x.new_empty(x.shape[:-1] + (n,))
    if addend is not None:
        if addend.shape != out.shape or addend.dtype != out.dtype:
            raise RuntimeError("addend must match the output")
        addend = addend.contiguous()
    _abi.check(_abi.load().parrot_decode_linear_bf16(
        ptr(x2), rows, k, ptr(weight), n, ptr(addend), ptr(out), _stream(x.device)),
        "parrot_decode_linear_bf16")
    return out


def decode_linear_supported(rows: int, k: int, n: int) -> bool:
    """Shapes parrot_decode_linear_bf16 takes."""
    return 1 <= rows <= 16 and k % 128 == 0 and k <= 2048 and rows * k * 2 <= 65536 and \
        n % 16 == 0


def mla_decode_out(context: Tensor, absorbed_output: Tensor,
                   addend: Tensor | None = None) -> Tensor:
    """bf16(context absorbed_output.float()^T) [b, 1, dim] (+ addend, a bf16
    sum) in one launch; context [b, H * r] fp32; cf.
    parrot/model.py:430-431."""
    if context.dtype != torch.float32 or context.device.type != "cuda":
        raise RuntimeError("HIP MLA decode output takes an fp32 ROCm context")
    _require(absorbed_output, "HIP MLA decode output")
    b, width = context.shape
    dim = absorbed_output.shape[0]
    if not absorbed_output.is_contiguous() or absorbed_output.shape[1] != width:
        raise RuntimeError("absorbed output map must be contiguous [dim, heads x latent]")
    context = context.contiguous()
    out = torch.empty((b, 1, dim), dtype=absorbed_output.dtype, device=context.device)
    if addend is not None:
        if addend.shape != out.shape or addend.dtype != out.dtype:
            raise RuntimeError("addend must match the [b, 1, dim] output")
        addend = addend.contiguous()
    _abi.check(_abi.load().parrot_mla_decode_out_bf16(
        ptr(context), b, width, ptr(absorbed_output), dim, ptr(addend), ptr(out),
        _stream(context.device)), "parrot_mla_decode_out_bf16")
    return out


def decode_attention_latent(q: Tensor, latent_new: Tensor, latent_cache: Tensor,
                            position: Tensor, heads: int, scale: float) -> Tensor:
    """One MLA decode step over the latent cache: store latent_new [b, 1, r]
    at position p and attend the fp32 absorbed queries q [b, 1, H * r] over
    latents 0 .. p (keys = values).  Returns the fp32 context [b, H * r]."""
    b, max_pos, r = latent_cache.shape
    if q.dtype != torch.float32 or q.device.type != "cuda" or torch.is_grad_enabled():
        raise RuntimeError("HIP latent decode attention takes fp32 ROCm queries without grad")
    _require(latent_new, "HIP latent decode attention")
    if q.numel() != b * heads * r or latent_new.shape != (b, 1, r):
        raise RuntimeError("latent decode shapes do not match the cache")
    if not latent_cache.is_contiguous():
        raise RuntimeError("latent cache must be contiguous")
    _check_position(position, q.device)
    q, latent_new = q.contiguous(), latent_new.contiguous()
    out = q.new_empty((b, heads * r))
    _abi.check(_abi.load().parrot_decode_attention_latent_f32(
        ptr(q), ptr(latent_new), ptr(latent_cache), ptr(position), b, heads, r, max_pos, scale,
        ptr(out), _stream(q.device)), "parrot_decode_attention_latent_f32")
    return out


# ---------------------------------------------------------------------------
# RMSNorm and Block AttnRes (cf. parrot/metal_moe.py:37-55, 419-477)
# ---------------------------------------------------------------------------

def rms_norm(module, x: Tensor) -> Tensor:
    """Inference RMSNorm for ROCm bf16 tensors."""
    _require(x, "HIP RMSNorm")
    x = x.contiguous()
    dim = x.shape[-1]
    rows = x.numel() // dim
    out = torch.empty_like(x)
    weight = module.weight
    if weight.dtype != x.dtype:
        raise RuntimeError("RMSNorm weight must match the input dtype")
    _abi.check(_abi.load().parrot_rms_norm_bf16(
        ptr(x), ptr(weight), ptr(out), rows, dim, float(module.eps), _stream(x.device)),
        "parrot_rms_norm_bf16")
    return out


_SourceArray = ctypes.c_void_p * MAX_DEPTH_SOURCES


def _depth(module, sources: list[Tensor], output_norm, router=None, logit_bias=None,
           pending=None):
    if not 1 <= len(sources) <= MAX_DEPTH_SOURCES:
        raise RuntimeError(f"HIP depth mixing supports one to {MAX_DEPTH_SOURCES} sources")
    first = sources[0]
    _require(first, "The HIP depth backend")
    dim = first.shape[-1]
    tokens = first.numel() // dim
    flat = []
    for s in sources:
        if s.shape != first.shape or s.dtype != first.dtype or s.device != first.device:
            raise RuntimeError("depth sources must share shape, dtype and device")
        flat.append(s.contiguous())
    array = _SourceArray(*([t.data_ptr() for t in flat] +
                           [flat[0].data_ptr()] * (MAX_DEPTH_SOURCES - len(flat))))
    out = torch.empty_like(flat[0])
    norm_w = None if output_norm is None else output_norm.weight
    mix_args = (ctypes.cast(array, ctypes.c_void_p), len(flat), ptr(module.query),
                ptr(module.norm.weight), float(module.norm.eps), ptr(norm_w),
                0.0 if output_norm is None else float(output_norm.eps), tokens, dim,
                ptr(out) if output_norm is None else None,
                None if output_norm is None else ptr(out))
    lib = _abi.load()
    if router is None:
        _abi.check(lib.parrot_depth_mix_bf16(*mix_args, _stream(first.device)),
                   "parrot_depth_mix_bf16")
        del flat  # the sources stay alive until the kernel is enqueued (it is)
        return out
    cfg = router.cfg
    router_w = router.router.weight
    if router_w.dtype != first.dtype or not router_w.is_contiguous():
        raise RuntimeError("router weight must be contiguous and match the input dtype")
    weights = torch.empty((tokens, 2), dtype=torch.float32, device=first.device)
    indices = torch.empty((tokens, 2), dtype=torch.int64, device=first.device)
    if logit_bias is not None:
        logit_bias = logit_bias.to(device=first.device, dtype=torch.float32).contiguous()
    if pending is None:
        _abi.check(lib.parrot_depth_mix_route_bf16(
            *mix_args, ptr(router_w), ptr(logit_bias), cfg.n_experts, ptr(weights), ptr(indices),
            _stream(first.device)), "parrot_depth_mix_route_bf16")
    else:
        contributions, base, resolved = pending
        if (contributions.dtype != torch.float32 or not contributions.is_contiguous() or
                contributions.numel() != tokens * PENDING_HEADS * dim or
                contributions.device != first.device):
            raise RuntimeError("contributions must be contiguous fp32 [tokens, 8, dim]")
        for t_ in (base, resolved):
            if t_ is not None and (t_.shape != first.shape or t_.dtype != first.dtype or
                                   not t_.is_contiguous() or t_.device != first.device):
                raise RuntimeError("base and resolved must be contiguous rows like the sources")
        _abi.check(lib.parrot_depth_mix_route_pending_bf16(
            *mix_args[:9], mix_args[10], ptr(router_w), ptr(logit_bias), cfg.n_experts,
            ptr(weights), ptr(indices), ptr(contributions), PENDING_HEADS, ptr(base),
            ptr(resolved), _stream(first.device)), "parrot_depth_mix_route_pending_bf16")
    del flat
    return out, RouteResult(None, weights, indices, None)


def embed_depth_mix_norm(ids: Tensor, table: Tensor, module, output_norm,
                         zeros: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """The forward's first launch: the embedding rows of ``ids`` [batch, T]
    (as ``table[ids]``, parrot/model.py:679) and ``depth_mix_norm(module,
    [rows], output_norm)`` (parrot/model.py:685-687), the same bits as the
    two steps; ``zeros`` (an fp32 tensor) is zero-filled by the same launch.
    Ids outside the table read its nearest row: the caller validates them."""
    _require(table, "The HIP depth backend")
    if ids.dtype != torch.int64 or ids.device != table.device or table.ndim != 2:
        raise RuntimeError("ids must be int64 on the table's device; table [vocab, dim]")
    if not table.is_contiguous():
        raise RuntimeError("embedding table must be contiguous")
    if zeros is not None and (zeros.dtype != torch.float32 or zeros.device != table.device or
                              not zeros.is_contiguous()):
        raise RuntimeError("zeros must be a contiguous fp32 tensor on the table's device")
    flat = ids.contiguous()
    vocab, dim = table.shape
    rows = torch.empty((*ids.shape, dim), dtype=table.dtype, device=table.device)
    out = torch.empty_like(rows)
    _abi.check(_abi.load().parrot_embed_depth_mix_bf16(
        ptr(flat), flat.numel(), ptr(table), vocab, dim, ptr(module.query),
        ptr(module.norm.weight), float(module.norm.eps), ptr(output_norm.weight),
        float(output_norm.eps), ptr(rows), ptr(out), ptr(zeros),
        0 if zeros is None else zeros.numel(), _stream(table.device)),
        "parrot_embed_depth_mix_bf16")
    return rows, out


def depth_mix(module, sources: list[Tensor]) -> Tensor:
    """Block AttnRes mix of 1..9 sources (cf. metal_depth_mix)."""
    return _depth(module, sources, None)


def depth_mix_norm(module, sources: list[Tensor], output_norm) -> Tensor:
    """Depth mix rounded to bf16, then the consumer RMSNorm, in one kernel
    (cf. metal_depth_mix_norm, for every token count)."""
    return _depth(module, sources, output_norm)


def depth_mix_norm_route(module, sources: list[Tensor], output_norm, moe: "MoE",
                         logit_bias: Tensor | None = None,
                         pending: tuple | None = None) -> tuple[Tensor, RouteResult]:
    """``depth_mix_norm`` of a MoE layer's input plus that layer's router
    top-2 on the result, in one kernel: at every token count the weights
    and indices equal ``route(moe, result)``'s bit for bit (no grouping, no
    router stats).  ``pending`` = (contributions fp32 [tokens, 8, dim], base
    or None, resolved): the last source is the deferred attention output
    bf16(base + bf16(sum of the contributions over heads)), made in the
    kernel and written to ``resolved`` (``sources[-1]`` only holds its
    place)."""
    if moe.cfg.top_k != 2 or moe.cfg.n_experts > MAX_EXPERTS:
        raise RuntimeError(f"HIP routing supports top-2 of at most {MAX_EXPERTS} experts")
    return _depth(module, sources, output_norm, router=moe, logit_bias=logit_bias,
                  pending=pending)
