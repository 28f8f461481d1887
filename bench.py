#!/usr/bin/env python3
"""Benchmark of the MI355X Parrot inference MoE path (one GPU).

Workload (the headline metric): the full default
Parrot model -- 16 layers, E=16 experts, top-2 + shared expert, Block
AttnRes, 32768-vocab tied head -- random-init with seed 2, bf16, router
statistics off, forward over batch 1 x 512 token ids drawn uniformly from
[0, 32768) (synthetic data).  MoE, RMSNorm and depth mixing run on the HIP
kernels (moe_backend="grouped_hip", depth_backend="hip"), and so do the
attention blocks and their projections; the embedding gather and the
vocabulary head GEMM are PyTorch-ROCm (hipBLASLt).

A step is one full forward.  The timed loop replays the forward captured in
a HIP graph (each replay recomputes everything from the static input ids);
the eager rate is reported beside it.  Per-kernel durations of the hot path
are measured with HIP events on the stream the kernels are launched on, at
the in-model shapes, and the dominant kernel's roofline fraction is
reported.  The CPU baseline is the fp32 CPU oracle of the reference's
``moe_backend="pytorch"`` forward on a bounded sample.

Prints one JSON line on stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "parrot-h200-worker_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBPS = 8000.0        # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
REFERENCE_TOK_S = 5250.0      # reference grouped_mps, same workload, Apple M4 Pro (README.md:43)
TOKENS = 512


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--kernel-iters", type=int, default=200)
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="approximate CPU time spent on the cpu_baseline sample")
    p.add_argument("--skip-cpu-baseline", action="store_true")
    p.add_argument("--skip-kernels", action="store_true")
    p.add_argument("--skip-sweep", action="store_true",
                   help="skip the token-count sweep of the per-kernel timings")
    p.add_argument("--skip-decode", action="store_true")
    p.add_argument("--sweep-only", action="store_true",
                   help="only the token-count sweep of the per-kernel timings (one JSON line)")
    p.add_argument("--pmc-workload", action="store_true",
                   help="only launch the counter workload: every hot-path kernel at C2, C3, "
                        "the C4 layer and T=65536, segments separated by a 16-byte marker copy")
    p.add_argument("--summarize-pmc", nargs="+", metavar="PASS_DIR",
                   help="(no GPU) turn the counter CSVs of the --pmc passes (A, B, C) over "
                        "--pmc-workload into profiles/counters_hot_path.json")
    p.add_argument("--summarize-steps", metavar="TRACE_DIR",
                   help="write the forward and decode kernel-trace summaries under profiles/ "
                        "from a rocprofv3 --kernel-trace run of bench.py --skip-kernels")
    p.add_argument("--summarize-trace", metavar="TRACE_DIR",
                   help="(no GPU) per-kernel durations of a rocprofv3 --kernel-trace run of "
                        "bench.py into profiles/kernel_trace_bench.json")
    return p.parse_args()


# ---------------------------------------------------------------------------
# per-kernel timing through the C ABI (no allocation inside the timed loop)
# ---------------------------------------------------------------------------

class StageBench:
    """Preallocated buffers for timing each C-ABI stage of one MoE layer."""

    def __init__(self, moe, x, logit_bias=None):
        import torch
        from parrot import _abi, hip_moe
        from parrot._abi import ptr
        self.torch, self.lib, self.ptr = torch, _abi.load(), ptr
        cfg = moe.cfg
        self.moe, self.x = moe, x.contiguous()
        self.T, self.dim = x.shape
        self.E, self.H, self.Hs = cfg.n_experts, cfg.expert_dim, cfg.shared_expert_dim
        self.C = hip_moe.capacity(self.T, self.E)
        self.bias = None if logit_bias is None else logit_bias.to(x.device, torch.float32)
        dev = x.device
        with torch.no_grad():
            self.routed = hip_moe.route(moe, self.x, False, logit_bias=self.bias)
            self.packed = hip_moe.pack_expert_weights(moe)
        g = self.routed.grouping
        self.g = g
        self.rws_bytes = self.lib.parrot_route_workspace_bytes(self.T, self.E)
        self.rws = torch.empty(max(self.rws_bytes, 256), dtype=torch.uint8, device=dev)
        self.ews_bytes = self.lib.parrot_experts_workspace_bytes(self.T, self.dim, self.H, self.Hs)
        self.ews = torch.empty(self.ews_bytes, dtype=torch.uint8, device=dev)
        self.out = torch.empty_like(self.x)
        self.stream = torch.cuda.current_stream(dev)
        self.s = self.stream.cuda_stream
        counts = g.counts.cpu()
        self.hit = int((counts > 0).sum())
        self.overflow = int(g.offsets[-1].item())
        # The forward's form at sizes the gate/up launch groups itself: the
        # top-2 ids (mode 1) or the route block table (mode 2) in; counts,
        # offsets and the hidden rows' ids out.
        self.group_mode = int(self.lib.parrot_experts_group_in_kernel(
            self.T, self.dim, self.E, self.H, self.Hs))
        self.in_kernel = self.group_mode != 0
        self.blocks = (torch.empty(((self.T + 15) // 16, 64), dtype=torch.uint8, device=dev)
                       if self.group_mode == 2 else None)
        i32 = dict(dtype=torch.int32, device=dev)
        self.g_counts = torch.empty(self.E, **i32)
        self.g_offsets = torch.empty(2 * self.E + 2, **i32)
        self.g_sorted = torch.empty(2 * self.T, **i32)
        self.ids = self.routed.indices.reshape(-1).contiguous()
        self.top2_ids = torch.empty_like(self.routed.indices)
        if self.blocks is not None:
            # The table gate_up_grouping reads when timed on its own.
            _abi.check(self.route_top2(), "parrot_route_top2_blocks_bf16")

    def route(self):
        p, r, g = self.ptr, self.routed, self.g
        return self.lib.parrot_route_bf16(
            p(self.x), p(self.moe.router.weight), p(self.bias), self.T, self.dim, self.E, self.C,
            None, None, p(r.weights), p(r.indices), p(g.positions), p(g.counts), p(g.offsets),
            p(g.perm), p(g.overflow), p(self.rws), self.rws_bytes, self.s)

    def route_top2(self):
        p, r = self.ptr, self.routed
        if self.blocks is not None:
            return self.lib.parrot_route_top2_blocks_bf16(
                p(self.x), p(self.moe.router.weight), p(self.bias), self.T, self.dim, self.E,
                p(r.weights), p(self.top2_ids), p(self.blocks), self.s)
        return self.lib.parrot_route_top2_bf16(
            p(self.x), p(self.moe.router.weight), p(self.bias), self.T, self.dim, self.E,
            p(r.weights), p(self.top2_ids), self.s)

    def layer(self):
        """The standalone MoE layer as MoE.inference runs it: top-2 + the
        grouping gate/up, down and combine where the gate/up launch groups
        in-kernel, else route + grouping, gate/up, down and combine."""
        steps = ((self.route_top2, self.gate_up_grouping_top2, self.down_sorted, self.combine)
                 if self.in_kernel else (self.route, self.gate_up, self.down, self.combine))
        for step in steps:
            rc = step()
            if rc:
                return rc
        return 0

    def gate_up_grouping_top2(self):
        p = self.ptr
        if self.blocks is not None:
            return self.gate_up_grouping()
        return self.lib.parrot_experts_gate_up_grouping_bf16(
            p(self.x), self.T, self.dim, self.E, self.H, self.Hs, self.C, p(self.top2_ids),
            p(self.g_counts), p(self.g_offsets), p(self.g_sorted), p(self.packed[0]),
            p(self.packed[2]), p(self.ews), self.ews_bytes, self.s)

    def layer_min_bytes(self):
        """Hit experts' weights once, the shared expert, the router, x in and
        out written (the layer's HBM floor)."""
        T, d, H, Hs, E = self.T, self.dim, self.H, self.Hs, self.E
        return (self.hit * 3 * d * H + 3 * d * Hs + E * d + 2 * T * d) * 2

    def layer_flops(self):
        return 2 * self.T * self.dim * self.E + self.flops_gate_up() + self.flops_down()

    def gate_up(self):
        p, g = self.ptr, self.g
        return self.lib.parrot_experts_gate_up_bf16(
            p(self.x), self.T, self.dim, self.E, self.H, self.Hs, self.C, p(g.counts),
            p(g.offsets), p(g.perm), p(g.overflow), p(self.packed[0]), p(self.packed[2]),
            p(self.ews), self.ews_bytes, self.s)

    def down(self):
        p, g = self.ptr, self.g
        return self.lib.parrot_experts_down_bf16(
            self.T, self.dim, self.E, self.H, self.Hs, self.C, p(g.counts), p(g.offsets),
            p(g.perm), p(g.overflow), p(self.routed.weights), p(self.packed[1]),
            p(self.packed[3]), p(self.ews), self.ews_bytes, self.s)

    def gate_up_grouping(self, weights=None):
        """``weights``: (routed gate/up, shared gate/up) packed copies to read
        in place of the layer's own (the cold-cache rotation)."""
        p = self.ptr
        gu, sh = (self.packed[0], self.packed[2]) if weights is None else weights
        if self.blocks is not None:
            return self.lib.parrot_experts_gate_up_grouping_blocks_bf16(
                p(self.x), self.T, self.dim, self.E, self.H, self.Hs, self.C, p(self.blocks),
                p(self.g_counts), p(self.g_offsets), p(self.g_sorted), p(gu), p(sh),
                p(self.ews), self.ews_bytes, self.s)
        return self.lib.parrot_experts_gate_up_grouping_bf16(
            p(self.x), self.T, self.dim, self.E, self.H, self.Hs, self.C, p(self.ids),
            p(self.g_counts), p(self.g_offsets), p(self.g_sorted), p(gu), p(sh),
            p(self.ews), self.ews_bytes, self.s)

    def with_x(self, x, stage):
        """A call of ``stage`` (a method name) reading token rows ``x`` (a copy
        of the layer's input) instead of the layer's own."""
        def call():
            own, self.x = self.x, x
            try:
                return getattr(self, stage)()
            finally:
                self.x = own
        return call

    def down_sorted(self):
        p = self.ptr
        return self.lib.parrot_experts_down_sorted_bf16(
            self.T, self.dim, self.E, self.H, self.Hs, self.C, p(self.g_counts),
            p(self.g_offsets), p(self.g_sorted), p(self.routed.weights), p(self.packed[1]),
            p(self.packed[3]), p(self.ews), self.ews_bytes, self.s)

    def combine(self):
        p = self.ptr
        return self.lib.parrot_experts_combine_bf16(self.T, self.dim, self.H, self.Hs, None,
                                                    p(self.out), p(self.ews), self.ews_bytes,
                                                    self.s)

    # algorithmic bytes / flops per launch
    def bytes_route(self):
        T, d, E = self.T, self.dim, self.E
        return T * d * 2 + E * d * 2 + 2 * T * (8 + 4 + 4) + E * 4 + E * self.C * 4 + self.overflow * 4

    def bytes_gate_up(self):
        T, d, H, Hs = self.T, self.dim, self.H, self.Hs
        return (self.hit * 2 * H * d + 2 * Hs * d + T * d + 2 * T * H + T * Hs) * 2

    def bytes_down(self):
        T, d, H, Hs = self.T, self.dim, self.H, self.Hs
        return (self.hit * d * H + d * Hs + 2 * T * H + T * Hs + 3 * T * d) * 2 + 2 * T * 4

    def bytes_grouping(self):
        """Extra bytes of the in-kernel grouping: ids (or the route block
        table) in, grouping out."""
        ids = 2 * self.T * 8 if self.blocks is None else self.blocks.numel()
        return ids + (3 * self.E + 2 + 2 * self.T) * 4

    def bytes_combine(self):
        return 3 * self.T * self.dim * 2 + self.T * self.dim * 2

    def flops_gate_up(self):
        return 2 * (2 * self.T) * 2 * self.H * self.dim + 2 * self.T * 2 * self.Hs * self.dim

    def flops_down(self):
        return 2 * (2 * self.T) * self.H * self.dim + 2 * self.T * self.Hs * self.dim


def event_time_us(fn, iters: int, stream) -> float:
    """Average duration of `fn`'s launches, HIP events on `stream`."""
    import torch
    for _ in range(5):
        rc = fn()
        if rc:
            raise RuntimeError(f"stage returned status {rc}")
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1000.0 / iters


def stage_time_us(fn, iters: int, stream, reps: int = 3) -> float:
    """The best of `reps` event_time_us loops: a stage entry is what the
    kernel takes, not a loop that a clock or power transition slowed."""
    return min(event_time_us(fn, iters, stream) for _ in range(reps))


# MI355X's memory-side cache (Infinity Cache): a loop that relaunches a kernel
# over the same buffers finds a working set below this size there, not in HBM.
MALL_BYTES = 256 << 20
COLD_ROTATION_BYTES = 512 << 20


def rotation(calls: list):
    """One callable that takes `calls` in turn: each launch reads its own
    copy of the inputs, last read len(calls) - 1 launches earlier."""
    turn = [0]

    def call():
        fn = calls[turn[0] % len(calls)]
        turn[0] += 1
        return fn()
    return call


def copies_for_cold(nbytes: int) -> int:
    """Input copies a rotation needs so that at least COLD_ROTATION_BYTES
    (twice the memory-side cache) are read between two reads of one copy."""
    return max(2, -(-COLD_ROTATION_BYTES // max(1, nbytes)))


def cold_time_us(calls: list, stream, laps: int = 2, reps: int = 3) -> float:
    """Average launch duration over a rotation of input copies (HIP events,
    best of `reps` loops of `laps` passes): every launch finds its inputs
    evicted from L2 and the memory-side cache, as a kernel inside the
    forward finds its layer's weights."""
    fn = rotation(calls)
    return min(event_time_us(fn, laps * len(calls), stream) for _ in range(reps))


# Attained peaks of this GPU (attained_peaks), once measured: every entry then
# also states its fraction of what the copy / MFMA-loop kernels reach.
ATTAINED: dict = {}


def entry(us: float, nbytes: int, flops: int | None = None, cold: bool = False) -> dict:
    """A kernel-table entry.  ``mall_resident``: the loop relaunched the
    kernel over the same buffers and they fit the memory-side cache, so the
    time is a warm one (reads served from that cache, not HBM); entries timed
    over a rotation of input copies (``cold``) read from HBM."""
    gbps = nbytes / (us * 1e-6) / 1e9
    out = {"us": round(us, 3), "bytes": int(nbytes), "gbps": round(gbps, 1),
           "hbm_frac": round(gbps / PEAK_HBM_GBPS, 4),
           "mall_resident": (not cold) and nbytes < MALL_BYTES}
    if cold:
        out["cold"] = True
    if ATTAINED.get("copy_gbps"):
        out["hbm_frac_attained"] = round(gbps / ATTAINED["copy_gbps"], 4)
    if flops is not None:
        tf = flops / (us * 1e-6) / 1e12
        out.update(flops=int(flops), tflops=round(tf, 2), mfma_frac=round(tf / PEAK_BF16_TFLOPS, 4))
        if ATTAINED.get("mfma_bf16_tflops"):
            out["mfma_frac_attained"] = round(tf / ATTAINED["mfma_bf16_tflops"], 4)
    return out


def attained_peaks() -> dict:
    """What this GPU reaches: the bf16 MFMA-loop microkernel at both MFMA
    shapes (4096 workgroups, register operands) and a 1 GiB device copy
    (this library's copy kernel and torch's copy_), HIP events, best of 3."""
    import ctypes

    import torch
    from parrot import _abi
    lib = _abi.load()
    s = torch.cuda.current_stream()
    res = {}
    out = torch.empty(4096 * 256, device="cuda")
    flops = ctypes.c_int64()
    for wide, iters, name in ((1, 2000, "mfma_32x32x16_tflops"), (0, 4000, "mfma_16x16x32_tflops")):
        def run():
            return lib.parrot_peak_mfma_bf16(wide, 4096, iters, out.data_ptr(), ctypes.byref(flops),
                                             s.cuda_stream)
        us = min(event_time_us(run, 3, s) for _ in range(3))
        res[name] = round(flops.value / (us * 1e-6) / 1e12, 1)
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    own = min(event_time_us(lambda: lib.parrot_peak_copy(src.data_ptr(), dst.data_ptr(), n, 8192,
                                                         s.cuda_stream), 5, s) for _ in range(3))

    def torch_copy():
        dst.copy_(src)
        return 0
    tc = min(event_time_us(torch_copy, 5, s) for _ in range(3))
    res["copy_kernel_gbps"] = round(2 * n / (own * 1e-6) / 1e9, 1)
    res["torch_copy_gbps"] = round(2 * n / (tc * 1e-6) / 1e9, 1)
    res["mfma_bf16_tflops"] = max(res["mfma_32x32x16_tflops"], res["mfma_16x16x32_tflops"])
    res["copy_gbps"] = max(res["copy_kernel_gbps"], res["torch_copy_gbps"])
    res["vendor"] = {"mfma_bf16_tflops": PEAK_BF16_TFLOPS, "hbm_gbps": PEAK_HBM_GBPS}
    # Latency floors of one launch in a dependent back-to-back chain, the
    # regime of every model-size kernel here: a 16-byte copy (one
    # workgroup), and copies of 1 / 8 / 24 MiB warm (the same buffer each
    # time: L2 and memory-side cache hits) and cold (rotating over 512 MiB of
    # buffers, twice the memory-side cache, so every read comes from HBM).
    floors = {"launch_16B_us": round(min(event_time_us(
        lambda: lib.parrot_peak_copy(src.data_ptr(), dst.data_ptr(), 16, 1, s.cuda_stream),
        200, s) for _ in range(3)), 2)}
    for mib in (1, 8, 24):
        nb = mib << 20
        blocks = max(64, min(8192, nb // 4096))
        floors[f"copy_{mib}MiB_warm_us"] = round(min(event_time_us(
            lambda: lib.parrot_peak_copy(src.data_ptr(), dst.data_ptr(), nb, blocks,
                                         s.cuda_stream), 100, s) for _ in range(3)), 2)
        slots = (512 << 20) // nb
        turn = [0]

        def cold():
            o = (turn[0] % slots) * nb
            turn[0] += 1
            return lib.parrot_peak_copy(src.data_ptr() + o, dst.data_ptr() + o, nb, blocks,
                                        s.cuda_stream)
        floors[f"copy_{mib}MiB_cold_us"] = round(min(event_time_us(cold, slots, s)
                                                     for _ in range(3)), 2)
    res["latency_floors"] = floors
    del src, dst, out
    torch.cuda.empty_cache()
    return res


def trace_marker(sb: "StageBench") -> None:
    """A 16-byte parrot_peak_copy on the stage stream: in a kernel trace of
    bench.py it opens the roofline kernel's timed loop (summarize_trace)."""
    from parrot import _abi
    buf = sb.torch.zeros(32, dtype=sb.torch.uint8, device=sb.x.device)
    _abi.check(sb.lib.parrot_peak_copy(sb.ptr(buf), sb.ptr(buf[16:]), 16, 1,
                                       sb.stream.cuda_stream), "trace marker")


def layer_kernels(moe, x, iters, logit_bias=None, mark_roofline=False
                  ) -> tuple[dict, "StageBench"]:
    sb = StageBench(moe, x, logit_bias)
    res = {
        "route_group": entry(stage_time_us(sb.route, iters, sb.stream), sb.bytes_route()),
        "gate_up": entry(stage_time_us(sb.gate_up, iters, sb.stream), sb.bytes_gate_up(),
                         sb.flops_gate_up()),
        "down": entry(stage_time_us(sb.down, iters, sb.stream), sb.bytes_down(), sb.flops_down()),
        "combine": entry(stage_time_us(sb.combine, iters, sb.stream), sb.bytes_combine()),
        "experts_hit": sb.hit,
        "overflow_assignments": sb.overflow,
        "capacity": sb.C,
    }
    if sb.in_kernel:
        # gate/up grouping first: down_sorted reads the grouping it writes.
        gu_bytes = sb.bytes_gate_up() + sb.bytes_grouping()
        if mark_roofline:
            # The roofline loop, cold: the launches rotate over copies of the
            # packed gate/up weights (>= 512 MiB read between two reads of a
            # copy), as the forward's launch finds its layer's weights in
            # HBM.  One timed loop between two marker copies: the kernel
            # trace summary takes exactly the dispatches after the first.
            w_bytes = (sb.packed[0].numel() * sb.packed[0].element_size() +
                       sb.packed[2].numel() * sb.packed[2].element_size())
            weights = [(sb.packed[0].clone(), sb.packed[2].clone())
                       for _ in range(copies_for_cold(w_bytes))]
            calls = [lambda w=w: sb.gate_up_grouping(w) for w in weights]
            trace_marker(sb)
            res["gate_up_grouping_cold"] = entry(
                event_time_us(rotation(calls), 4 * len(calls), sb.stream), gu_bytes,
                sb.flops_gate_up(), cold=True)
            res["gate_up_grouping_cold"]["weight_copies"] = len(calls)
            trace_marker(sb)
            del calls, weights
        res["gate_up_grouping"] = entry(stage_time_us(sb.gate_up_grouping, iters, sb.stream),
                                        gu_bytes, sb.flops_gate_up())
        res["down_sorted"] = entry(stage_time_us(sb.down_sorted, iters, sb.stream),
                                   sb.bytes_down() + (3 * sb.E + 2) * 4, sb.flops_down())
        res["route_top2"] = entry(stage_time_us(sb.route_top2, iters, sb.stream),
                                  sb.T * sb.dim * 2 + sb.E * sb.dim * 2 + sb.T * 2 * (8 + 4) +
                                  (0 if sb.blocks is None else sb.blocks.numel()))
    # The whole standalone layer, back to back on one stream, against the
    # layer's HBM floor (hit experts' weights once + x in + out) and its flops.
    layer = entry(stage_time_us(sb.layer, iters, sb.stream), sb.layer_min_bytes(), sb.layer_flops())
    layer["launches"] = (
        "route_top2 + gate_up(grouping in-kernel) + down + combine" if sb.group_mode == 1 else
        "route_top2(+block table) + gate_up(grouping in-kernel) + down + combine"
        if sb.group_mode == 2 else "route(+grouping) + gate_up + down + combine")
    layer["tokens_per_s"] = round(sb.T / (layer["us"] * 1e-6), 1)
    res["layer"] = layer
    return res, sb


def norm_kernels(model, iters) -> dict:
    import ctypes

    import torch
    from parrot import _abi
    from parrot._abi import ptr
    lib = _abi.load()
    dev = torch.device("cuda:0")
    d = model.config.dim
    x = torch.randn(TOKENS, d, device=dev).bfloat16()
    out = torch.empty_like(x)
    norm = model.blocks[0].attention_norm
    s = torch.cuda.current_stream(dev)
    rms_us = stage_time_us(lambda: lib.parrot_rms_norm_bf16(ptr(x), ptr(norm.weight), ptr(out),
                                                            TOKENS, d, 1e-6, s.cuda_stream),
                           iters, s)
    srcs = [torch.randn(TOKENS, d, device=dev).bfloat16() for _ in range(9)]
    arr = (ctypes.c_void_p * 9)(*[t.data_ptr() for t in srcs])
    mix = model.depth_mix[-1]
    depth_us = stage_time_us(
        lambda: lib.parrot_depth_mix_bf16(ctypes.cast(arr, ctypes.c_void_p), 9, ptr(mix.query),
                                          ptr(mix.norm.weight), 1e-6, ptr(norm.weight), 1e-6,
                                          TOKENS, d, None, ptr(out), s.cuda_stream), iters, s)
    return {
        "rms_norm": entry(rms_us, 2 * TOKENS * d * 2 + d * 2),
        "depth_mix_norm_s9": entry(depth_us, 9 * TOKENS * d * 2 + 3 * d * 2 + TOKENS * d * 2),
    }


# ---------------------------------------------------------------------------
# CPU baseline: the fp32 CPU oracle of the reference pytorch forward
# ---------------------------------------------------------------------------

def cpu_baseline(model, ids, seconds: float) -> dict:
    import torch

    from oracle import parrot_fp32
    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    oracle = parrot_fp32.ParrotFP32(model.config, model.state_dict())
    cpu_ids = ids.cpu()
    with torch.no_grad():
        oracle.forward(cpu_ids)  # warmup
        samples = []
        t_start = time.perf_counter()
        while len(samples) < 3 or (time.perf_counter() - t_start < seconds and len(samples) < 200):
            t0 = time.perf_counter()
            oracle.forward(cpu_ids)
            samples.append(time.perf_counter() - t0)
    med = statistics.median(samples)
    cpu_model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(TOKENS / med, 2), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"{len(samples)} fp32 CPU forwards of the same 1x512 workload "
                      f"(oracle/parrot_fp32.py, the reference pytorch path), median "
                      f"{med * 1e3:.1f} ms; cpu_count={os.cpu_count()}; {cpu_model}"}


# ---------------------------------------------------------------------------
# token-count sweep, decode, CPU layer baselines
# ---------------------------------------------------------------------------

SWEEP_TOKENS = (512, 4096, 16384, 65536)
COLD_SWEEP_TOKENS = 16384  # from here the sweep also times the bandwidth kernels cold


def sweep_kernels(moe, iters: int) -> dict:
    """Every hot-path kernel of one E=16 MoE layer (block 0's weights) plus
    RMSNorm and the 9-source depth mix, at growing token counts: where the
    per-launch fixed cost stops dominating, the bandwidth kernels approach
    their HBM asymptote and the expert GEMMs become MFMA-bound."""
    import ctypes

    import torch
    from parrot import _abi
    from parrot._abi import ptr
    lib = _abi.load()
    dev = torch.device("cuda:0")
    d = moe.cfg.dim
    gen = torch.Generator(device=dev).manual_seed(7)
    out = {}
    for T in SWEEP_TOKENS:
        n = max(10, iters if T <= 4096 else iters // 4)
        x = torch.randn(T, d, device=dev, generator=gen).bfloat16()
        res, sb = layer_kernels(moe, x, n)
        y = torch.empty_like(x)
        s = torch.cuda.current_stream(dev)
        w = torch.ones(d, device=dev, dtype=torch.bfloat16)
        res["rms_norm"] = entry(stage_time_us(
            lambda: lib.parrot_rms_norm_bf16(ptr(x), ptr(w), ptr(y), T, d, 1e-6, s.cuda_stream),
            n, s), 2 * T * d * 2 + d * 2)
        srcs = [torch.randn(T, d, device=dev, generator=gen).bfloat16() for _ in range(9)]
        arr = (ctypes.c_void_p * 9)(*[t.data_ptr() for t in srcs])
        q = torch.randn(d, device=dev, generator=gen).bfloat16()

        def mix(a):
            return lambda: lib.parrot_depth_mix_bf16(ctypes.cast(a, ctypes.c_void_p), 9, ptr(q),
                                                     ptr(w), 1e-6, ptr(w), 1e-6, T, d, None,
                                                     ptr(y), s.cuda_stream)
        mix_bytes = 9 * T * d * 2 + 3 * d * 2 + T * d * 2
        res["depth_mix_norm_s9"] = entry(stage_time_us(mix(arr), n, s), mix_bytes)
        if T >= COLD_SWEEP_TOKENS:
            # Cold: every launch reads its own copy of the inputs (rotations
            # over >= 512 MiB), so the bandwidth kernels' fractions are HBM's.
            xs = [x.clone() for _ in range(copies_for_cold(T * d * 2))]
            res["route_group_cold"] = entry(cold_time_us(
                [sb.with_x(xk, "route") for xk in xs], s), sb.bytes_route(), cold=True)
            res["route_top2_cold"] = entry(cold_time_us(
                [sb.with_x(xk, "route_top2") for xk in xs], s),
                T * d * 2 + sb.E * d * 2 + T * 2 * (8 + 4), cold=True)
            res["rms_norm_cold"] = entry(cold_time_us(
                [lambda xk=xk: lib.parrot_rms_norm_bf16(ptr(xk), ptr(w), ptr(y), T, d, 1e-6,
                                                        s.cuda_stream) for xk in xs], s),
                2 * T * d * 2 + d * 2, cold=True)
            del xs
            sets = [[t.clone() for t in srcs] for _ in range(copies_for_cold(9 * T * d * 2) - 1)]
            arrs = [arr] + [(ctypes.c_void_p * 9)(*[t.data_ptr() for t in st]) for st in sets]
            res["depth_mix_norm_s9_cold"] = entry(cold_time_us([mix(a) for a in arrs], s),
                                                  mix_bytes, cold=True)
            del sets, arrs
        out[f"T{T}"] = res
        del sb, srcs, x, y
        torch.cuda.empty_cache()
    return out


def decode_bench(model, steps: int = 16) -> dict:
    """prefill a 128-token prompt (seed 3), then `steps`
    greedy decode steps, at batch 1, 2, 4 and 8 (4096-position caches):
    eager `decode_next` steps, and the same steps replayed from one captured
    HIP graph (`parrot.decode_graph.DecodeGraph`; its one-time capture is
    reported separately)."""
    import torch
    from parrot.decode_graph import DecodeGraph
    dev = torch.device("cuda:0")
    out = {}
    for b in (1, 2, 4, 8):
        prompt = torch.randint(0, 32768, (b, 128),
                               generator=torch.Generator().manual_seed(3)).to(dev)
        with torch.inference_mode():
            for _ in range(2):  # warm the allocator and kernels
                logits, state = model.prefill(prompt)
                nxt = logits[:, -1].argmax(-1, keepdim=True)
                for _ in range(2):
                    nxt, state = model.decode_next(nxt, state)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            logits, state = model.prefill(prompt)
            first = logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            nxt = first
            for _ in range(steps):
                nxt, state = model.decode_next(nxt, state)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            eager_tokens = nxt.clone()

            logits, state = model.prefill(prompt)
            torch.cuda.synchronize()
            t3 = time.perf_counter()
            graph = DecodeGraph(model, state)
            torch.cuda.synchronize()
            t4 = time.perf_counter()
            nxt = first
            for _ in range(steps):
                nxt = graph.step(nxt)
            torch.cuda.synchronize()
            t5 = time.perf_counter()
            if not torch.equal(nxt, eager_tokens):
                raise RuntimeError("graph-replayed decoding differs from eager decoding")
            del graph
        out[f"b{b}"] = {"prefill_ms": round((t1 - t0) * 1e3, 3),
                        "eager_decode_ms_per_step": round((t2 - t1) * 1e3 / steps, 3),
                        "eager_decode_tokens_per_s": round(b * steps / (t2 - t1), 1),
                        "eager_generation_tokens_per_s": round(b * steps / (t2 - t0), 1),
                        "graph_capture_ms": round((t4 - t3) * 1e3, 1),
                        "graph_decode_ms_per_step": round((t5 - t4) * 1e3 / steps, 3),
                        "graph_decode_tokens_per_s": round(b * steps / (t5 - t4), 1),
                        "graph_generation_tokens_per_s": round(
                            b * steps / ((t1 - t0) + (t5 - t4)), 1)}
    return out


def cpu_layer_baselines(seconds: float) -> dict:
    """The fp32 CPU oracle of one MoE layer (the reference's pytorch loop) at
    BASELINE configs 2 and 3, tokens/s."""
    import torch

    from oracle import layers
    out = {}
    for name, tokens, skew in (("C2_T256_E32", 256, False), ("C3_T4096_E32_skew", 4096, True)):
        moe, x, bias = _layer_case(tokens, skew, device="cpu", dtype=torch.float32)
        sd = {k: v.detach() for k, v in moe.state_dict().items()}
        experts = [(sd[f"experts.{e}.gate.weight"], sd[f"experts.{e}.up.weight"],
                    sd[f"experts.{e}.down.weight"]) for e in range(32)]
        shared = (sd["shared.gate.weight"], sd["shared.up.weight"], sd["shared.down.weight"])
        bias_np = None if bias is None else bias.numpy()
        with torch.no_grad():
            layers.moe_layer(x, sd["router.weight"], experts, shared, bias_np)
            samples = []
            t_start = time.perf_counter()
            while len(samples) < 3 or (time.perf_counter() - t_start < seconds / 2
                                       and len(samples) < 20):
                t0 = time.perf_counter()
                layers.moe_layer(x, sd["router.weight"], experts, shared, bias_np)
                samples.append(time.perf_counter() - t0)
        med = statistics.median(samples)
        out[name] = {"tokens_per_s": round(tokens / med, 1), "median_ms": round(med * 1e3, 3),
                     "runs": len(samples), "threads": torch.get_num_threads()}
    return out


# ---------------------------------------------------------------------------
# HBM traffic of the dominant kernel, from the counter passes below
# ---------------------------------------------------------------------------

TRAFFIC_KERNEL = "grouped_gemm_stream_kernel<32, 32, 4, 1, 1>"
TRAFFIC_SEGMENT = "C4_layer_T512_E16: gate/up grouping in-kernel"
CALIBRATION_ELEMS = 1 << 27       # bf16: 256 MiB read + 256 MiB written per launch


def load_traffic() -> int | None:
    """HBM bytes per launch of the roofline kernel, from the committed
    counter summary of every hot-path kernel."""
    counters = load_json(PMC_FILE)
    if counters and TRAFFIC_SEGMENT in counters.get("segments", {}):
        return counters["segments"][TRAFFIC_SEGMENT]["hbm_bytes"]
    return None


# ---------------------------------------------------------------------------
# Counter evidence for every hot-path kernel (three rocprofv3 --pmc passes)
# ---------------------------------------------------------------------------

PMC_FILE = ROOT / "profiles" / "counters_hot_path.json"
PMC_MANIFEST = "gpurun_out/pmc_manifest.json"
PMC_REPEATS = 5
PMC_PASSES = {
    "A": "FETCH_SIZE SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE",
    "B": "WRITE_SIZE",
    # L2 -> CU reads: requests from the vector L1s to the L2s, and L2 hits
    # and misses (the weights' re-reads by row tiles land here, not in HBM).
    "C": "TCP_TCC_READ_REQ_sum TCC_HIT_sum TCC_MISS_sum",
}
PMC_COMMANDS = [f"rocprofv3 --pmc {c} -f csv -d gpurun_out/pmc_{k} -o pmc "
                f"-- python3 bench.py --pmc-workload" for k, c in PMC_PASSES.items()] + [
    "python3 bench.py --summarize-pmc gpurun_out/pmc_A gpurun_out/pmc_B gpurun_out/pmc_C"]
MARKER_KERNEL = ("parrot", "copy_kernel")  # a 16-byte parrot_peak_copy opens every segment


def pmc_workload() -> None:
    """The dispatches the --pmc passes count, in segments: a marker copy, then
    PMC_REPEATS launches of one stage.  Calibration first (torch.neg over a
    known byte count, the MFMA loop over a known flop count), then route,
    grouping, gate/up, down and combine at C2, C3, block 0's input of the C4
    forward and T=65536 (E=16), RMSNorm and the 9-source depth mix at 512 and
    65536 tokens.  Writes the segment list to PMC_MANIFEST."""
    import ctypes

    import torch
    from parrot import _abi
    from parrot._abi import ptr
    lib = _abi.load()
    model, _, captured = build_model()
    s = torch.cuda.current_stream()
    moe0 = model.blocks[0].moe
    benches = {"C4_layer_T512_E16": StageBench(moe0, captured["x"])}
    for name, tokens, skew in (("C2_T256_E32", 256, False), ("C3_T4096_E32_skew", 4096, True)):
        moe, x, bias = _layer_case(tokens, skew)
        benches[name] = StageBench(moe, x, bias)
    big = torch.randn(65536, moe0.cfg.dim, device="cuda",
                      generator=torch.Generator(device="cuda").manual_seed(7)).bfloat16()
    benches["T65536_E16"] = StageBench(moe0, big)
    d = moe0.cfg.dim
    norm_cases = {}
    for T in (512, 65536):
        x = torch.randn(T, d, device="cuda").bfloat16()
        srcs = [torch.randn(T, d, device="cuda").bfloat16() for _ in range(9)]
        arr = (ctypes.c_void_p * 9)(*[t.data_ptr() for t in srcs])
        norm_cases[T] = (x, torch.empty_like(x), srcs, arr)
    w = torch.ones(d, device="cuda", dtype=torch.bfloat16)
    q = torch.randn(d, device="cuda").bfloat16()
    calib_src = torch.ones(CALIBRATION_ELEMS, dtype=torch.bfloat16, device="cuda")
    calib_dst = torch.empty_like(calib_src)
    loop_out = torch.empty(1024 * 256, device="cuda")
    loop_flops = ctypes.c_int64()
    mark_a = torch.zeros(16, dtype=torch.uint8, device="cuda")
    mark_b = torch.empty_like(mark_a)
    torch.cuda.synchronize()

    manifest = []

    def segment(label, fn, nbytes=None, flops=None):
        _abi.check(lib.parrot_peak_copy(ptr(mark_a), ptr(mark_b), 16, 1, s.cuda_stream), "marker")
        for _ in range(PMC_REPEATS):
            rc = fn()
            if rc:
                raise RuntimeError(f"{label}: status {rc}")
        manifest.append({"label": label, "bytes": nbytes, "flops": flops})

    def neg():
        torch.neg(calib_src, out=calib_dst)
        return 0

    segment("calibration: torch.neg bf16", neg, 2 * CALIBRATION_ELEMS * 2)
    segment("calibration: MFMA loop 32x32x16",
            lambda: lib.parrot_peak_mfma_bf16(1, 1024, 500, ptr(loop_out), ctypes.byref(loop_flops),
                                              s.cuda_stream))
    manifest[-1]["flops"] = loop_flops.value
    for cfg, sb in benches.items():
        segment(f"{cfg}: route + grouping", sb.route, sb.bytes_route())
        segment(f"{cfg}: route top-2", sb.route_top2,
                sb.T * sb.dim * 2 + sb.E * sb.dim * 2 + sb.T * 2 * (8 + 4))
        if sb.in_kernel:
            segment(f"{cfg}: gate/up grouping in-kernel", sb.gate_up_grouping,
                    sb.bytes_gate_up() + sb.bytes_grouping(), sb.flops_gate_up())
            segment(f"{cfg}: down (in-kernel grouping)", sb.down_sorted,
                    sb.bytes_down() + (3 * sb.E + 2) * 4, sb.flops_down())
        else:
            segment(f"{cfg}: gate/up", sb.gate_up, sb.bytes_gate_up(), sb.flops_gate_up())
            segment(f"{cfg}: down", sb.down, sb.bytes_down(), sb.flops_down())
        segment(f"{cfg}: combine", sb.combine, sb.bytes_combine())
    for T, (x, y, srcs, arr) in norm_cases.items():
        segment(f"T{T}: rms_norm",
                lambda: lib.parrot_rms_norm_bf16(ptr(x), ptr(w), ptr(y), T, d, 1e-6, s.cuda_stream),
                2 * T * d * 2 + d * 2)
        segment(f"T{T}: depth mix + norm, 9 sources",
                lambda: lib.parrot_depth_mix_bf16(ctypes.cast(arr, ctypes.c_void_p), 9, ptr(q),
                                                  ptr(w), 1e-6, ptr(w), 1e-6, T, d, None, ptr(y),
                                                  s.cuda_stream),
                9 * T * d * 2 + 3 * d * 2 + T * d * 2)
    torch.cuda.synchronize()
    Path(PMC_MANIFEST).parent.mkdir(parents=True, exist_ok=True)
    Path(PMC_MANIFEST).write_text(json.dumps(manifest, indent=1))
    print(json.dumps({"pmc_workload": "done", "segments": len(manifest),
                      "repeats": PMC_REPEATS}), flush=True)


def _dispatches(directory: str) -> list[dict]:
    """Per-dispatch rows (kernel, counters, duration) of a counter_collection
    CSV in dispatch order."""
    import csv
    by_id: dict[int, dict] = {}
    for path in sorted(Path(directory).rglob("*counter_collection.csv")):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                key = int(r["Dispatch_Id"])
                d = by_id.setdefault(key, {"kernel": r["Kernel_Name"], "counters": {},
                                           "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
                d["counters"][r["Counter_Name"]] = float(r["Counter_Value"])
    return [by_id[k] for k in sorted(by_id)]


def _segments(rows: list[dict]) -> list[list[dict]]:
    segs, cur = [], None
    for r in rows:
        if all(part in r["kernel"] for part in MARKER_KERNEL):
            cur = []
            segs.append(cur)
        elif cur is not None:
            cur.append(r)
    return segs


def summarize_pmc(dir_a: str, dir_b: str, dir_c: str | None = None) -> dict:
    manifest = json.loads(Path(PMC_MANIFEST).read_text())
    seg_a, seg_b = _segments(_dispatches(dir_a)), _segments(_dispatches(dir_b))
    seg_c = _segments(_dispatches(dir_c)) if dir_c else None
    if len(seg_a) < len(manifest) or len(seg_b) < len(manifest) or (
            seg_c is not None and len(seg_c) < len(manifest)):
        raise SystemExit(f"found {len(seg_a)} / {len(seg_b)} segments for {len(manifest)} labels")
    seg_a, seg_b = seg_a[-len(manifest):], seg_b[-len(manifest):]
    if seg_c is not None:
        seg_c = seg_c[-len(manifest):]

    def per_launch(seg, counter):
        return sum(r["counters"].get(counter, 0.0) for r in seg) / PMC_REPEATS

    # Calibration: counter KiB per byte moved, MFMA ops and busy cycles per flop.
    calib = 2 * CALIBRATION_ELEMS  # bytes each way
    fetch_scale = calib / 1024 / per_launch(seg_a[0], "FETCH_SIZE")
    write_scale = calib / 1024 / per_launch(seg_b[0], "WRITE_SIZE")
    loop = seg_a[1]
    loop_flops = manifest[1]["flops"]
    flop_per_mop = loop_flops / per_launch(loop, "SQ_INSTS_VALU_MFMA_MOPS_BF16")
    loop_busy = per_launch(loop, "SQ_VALU_MFMA_BUSY_CYCLES") / per_launch(loop, "GRBM_GUI_ACTIVE")
    loop_ns = sum(r["ns"] for r in loop) / PMC_REPEATS
    # L2 -> CU: bytes per TCP -> TCC read request, from the calibration read.
    req_bytes = (calib / per_launch(seg_c[0], "TCP_TCC_READ_REQ_sum")
                 if seg_c is not None else None)
    entries = {}
    for i, (m, a, b) in enumerate(list(zip(manifest, seg_a, seg_b))[2:], start=2):
        ns = sum(r["ns"] for r in a) / PMC_REPEATS
        fetch = per_launch(a, "FETCH_SIZE") * fetch_scale * 1024
        write = per_launch(b, "WRITE_SIZE") * write_scale * 1024
        e = {"kernels": sorted({_short_kernel(r["kernel"]) for r in a}),
             "us_under_pmc": round(ns / 1e3, 3),
             "fetch_bytes": int(fetch), "write_bytes": int(write),
             "hbm_bytes": int(fetch + write),
             "hbm_gbps": round((fetch + write) / ns, 1) if ns else None}
        if m["bytes"]:
            e["algorithmic_bytes"] = m["bytes"]
            e["traffic_over_algorithmic"] = round((fetch + write) / m["bytes"], 3)
        mops = per_launch(a, "SQ_INSTS_VALU_MFMA_MOPS_BF16")
        if m["flops"] and mops:
            e["algorithmic_flops"] = m["flops"]
            e["mfma_flops_counted"] = int(mops * flop_per_mop)
            e["mfma_tflops"] = round(mops * flop_per_mop / ns / 1e3, 1)
            busy = per_launch(a, "SQ_VALU_MFMA_BUSY_CYCLES") / per_launch(a, "GRBM_GUI_ACTIVE")
            e["mfma_busy_vs_loop"] = round(busy / loop_busy, 4)
        if seg_c is not None:
            c = seg_c[i]
            l2_read = per_launch(c, "TCP_TCC_READ_REQ_sum") * req_bytes
            hit, miss = per_launch(c, "TCC_HIT_sum"), per_launch(c, "TCC_MISS_sum")
            e["l2_to_cu_read_bytes"] = int(l2_read)
            if m["bytes"]:
                e["l2_reads_over_algorithmic"] = round(l2_read / m["bytes"], 3)
            e["l2_hit_rate"] = round(hit / (hit + miss), 4) if hit + miss else None
        entries[m["label"]] = e
    summary = {
        "what": "per-launch HBM bytes (FETCH_SIZE, WRITE_SIZE), MFMA counters and L2 -> CU "
                "read bytes (TCP_TCC_READ_REQ) with the L2 hit rate of every hot-path kernel, "
                "median workload of PMC_REPEATS launches per segment",
        "calibration": {
            "fetch_scale": round(fetch_scale, 4), "write_scale": round(write_scale, 4),
            "bytes_each_way": calib, "kernel": "torch.neg bf16, %d elements" % CALIBRATION_ELEMS,
            "bytes_per_tcp_tcc_read_req": round(req_bytes, 2) if req_bytes else None,
            "flop_per_mfma_op": round(flop_per_mop, 3),
            "mfma_loop": {"flops": loop_flops, "us_under_pmc": round(loop_ns / 1e3, 2),
                          "tflops": round(loop_flops / loop_ns / 1e3, 1),
                          "busy_cycles_over_gui_active": round(loop_busy, 4)}},
        "segments": entries,
        "commands": PMC_COMMANDS,
    }
    PMC_FILE.write_text(json.dumps(summary, indent=1) + "\n")
    return summary


TRACE_FILE = ROOT / "profiles" / "kernel_trace_bench.json"
BENCH_FILE = ROOT / "profiles" / "bench_forward_bs1x512.json"


def summarize_trace(directory: str) -> dict:
    """Per-kernel dispatch counts and mean durations of a rocprofv3
    --kernel-trace run of bench.py; for the roofline kernel, the dispatches
    of its timed back-to-back loop (the run after bench.py's marker copy)
    apart from those inside the graph-replayed forwards (runs of < 20)."""
    import csv
    rows = []
    for path in sorted(Path(directory).rglob("*kernel_trace.csv")):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"],
                             int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    rows.sort()
    stats: dict[str, list[int]] = {}
    for _, name, ns in rows:
        stats.setdefault(name, []).append(ns)
    # The timed loop: the run of the roofline kernel right after the 16-byte
    # marker copy bench.py issues before it (its 5 warm-up launches
    # included); the in-forward dispatches: its runs shorter than 20.
    loop, graph, run, after_marker, prev = [], [], [], False, ""
    for _, name, ns in rows + [(None, "", 0)]:
        if TRAFFIC_KERNEL in name:
            if not run:
                after_marker = all(part in prev for part in MARKER_KERNEL)
            run.append(ns)
            prev = name
            continue
        if run and after_marker and not loop:
            loop.extend(run)
        elif len(run) < 20:
            graph.extend(run)
        run, prev = [], name
    summary = {
        "roofline_kernel": TRAFFIC_KERNEL,
        "loop_dispatches": len(loop),
        "loop_mean_us": round(statistics.mean(loop) / 1e3, 3) if loop else None,
        "in_forward_dispatches": len(graph),
        "in_forward_mean_us": round(statistics.mean(graph) / 1e3, 3) if graph else None,
        "kernels": {n[:160]: {"calls": len(v), "mean_us": round(statistics.mean(v) / 1e3, 3),
                              "total_us": round(sum(v) / 1e3, 1)}
                    for n, v in sorted(stats.items(), key=lambda kv: -sum(kv[1]))[:40]},
        "command": "rocprofv3 --kernel-trace --stats -f csv -d gpurun_out/bench_trace -o bench "
                   "-- python3 bench.py --skip-cpu-baseline --skip-decode; "
                   "python3 bench.py --summarize-trace gpurun_out/bench_trace",
    }
    TRACE_FILE.write_text(json.dumps(summary, indent=1) + "\n")
    return summary


def _short_kernel(name: str) -> str:
    """A kernel name without its argument list and namespaces."""
    n = name[5:] if name.startswith("void ") else name
    for ns in ("parrot::(anonymous namespace)::", "(anonymous namespace)::"):
        n = n.replace(ns, "")
    depth, cut = 0, len(n)
    for i, ch in enumerate(n):  # the argument list: the first '(' outside <...>
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    return n[:cut][:72]


def _step_table(steps: list[list[dict]]) -> tuple[str, float, float, float]:
    """Markdown table of per-kernel time over `steps` (lists of dispatches),
    with the launches, kernel time and first-start-to-last-end per step."""
    per: dict[tuple, list[int]] = {}
    for st in steps:
        for r in st:
            per.setdefault((_short_kernel(r["name"]), r["gx"], r["gy"], r["wg"]), []).append(r["ns"])
    n = len(steps)
    busy = sum(r["ns"] for st in steps for r in st) / n / 1e3
    span = sum(st[-1]["end"] - st[0]["start"] for st in steps) / n / 1e3
    launches = sum(len(st) for st in steps) / n
    lines = ["| kernel | grid x | grid y | wg | per step | mean us | median us | min us | "
             "us per step | share % |", "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for (name, gx, gy, wg), v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        tot = sum(v) / n / 1e3
        lines.append(f"| `{name}` | {gx} | {gy} | {wg} | {len(v) / n:g} | "
                     f"{statistics.mean(v) / 1e3:.2f} | {statistics.median(v) / 1e3:.2f} | "
                     f"{min(v) / 1e3:.2f} | {tot:.1f} | {100 * tot / busy:.1f} |")
    return "\n".join(lines), launches, busy, span


def summarize_steps(directory: str, out_dir: Path | None = None) -> str:
    """Per-kernel time of the graph-replayed forwards and decode steps in a
    rocprofv3 --kernel-trace run of `bench.py --skip-cpu-baseline
    --skip-kernels`: profiles/forward_bs1x512_kernel_trace.md and
    profiles/decode_graph_kernel_trace.md."""
    import csv
    rows = []
    for path in sorted(Path(directory).rglob("*kernel_trace.csv")):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append({"id": int(r["Dispatch_Id"]), "name": r["Kernel_Name"],
                             "start": int(r["Start_Timestamp"]), "end": int(r["End_Timestamp"]),
                             "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"]),
                             "gx": int(r["Grid_Size_X"]), "gy": int(r["Grid_Size_Y"]),
                             "wg": int(r["Workgroup_Size_X"])})
    rows.sort(key=lambda r: r["id"])
    command = ("rocprofv3 --kernel-trace --stats -f csv -d gpurun_out/prof_steps -o steps -- "
               "python3 -u bench.py --skip-cpu-baseline --skip-kernels\n"
               "python3 bench.py --summarize-steps gpurun_out/prof_steps")
    bench = load_json(BENCH_FILE) or {}
    out_dir = ROOT / "profiles" if out_dir is None else Path(out_dir)
    # Forwards: from one bs1 x 512 first launch (the embedding gather with
    # the first module's input, one workgroup per token) to the next; the
    # timed graph replays are the last `steps` of the most common launch count.
    starts = [i for i, r in enumerate(rows)
              if "embed_mix_kernel" in r["name"] and r["gx"] // r["wg"] == TOKENS]
    segs = [rows[a:b] for a, b in zip(starts, starts[1:] + [len(rows)])]
    counts = [len(sg) for sg in segs]
    mode = max(set(counts), key=counts.count) if counts else 0
    fwd = [sg for sg in segs if len(sg) == mode][-bench.get("steps", 20):]
    table, launches, busy, span = _step_table(fwd) if fwd else ("(no forwards)", 0, 0, 0)
    ms = bench.get("ms_per_step")
    (out_dir / "forward_bs1x512_kernel_trace.md").write_text(
        "# Kernel trace: Parrot bf16 forward, batch 1 x 512 (HIP-graph replay)\n\n"
        "Command (GPU box, repo root):\n\n```\n" + command + "\n```\n\n"
        f"The last {len(fwd)} forwards of the trace (the timed graph replays), split at each "
        f"forward's first launch (embedding rows and first module input).  Per forward: {launches:g} launches, {busy:.1f} us of "
        f"kernel time, {span:.1f} us from the first launch's start to the last one's end"
        + (f" (the committed bench line: {ms * 1e3:.1f} us per step)" if ms else "")
        + ".  Durations in us (End - Start), under the profiler.\n\n" + table + "\n")
    # Decode steps: each ends with the vocabulary argmax reduce; the batch is
    # the decode attention kernel's grid y; the last 16 steps of each batch
    # size are the graph replays.
    steps, cur = [], []
    for r in rows:
        cur.append(r)
        if "vocab_argmax_reduce" in r["name"]:
            steps.append(cur)
            cur = []
    by_batch: dict[int, list] = {}
    for st in steps:
        att = [r for r in st if "decode_attention_kernel" in r["name"]]
        if att:
            by_batch.setdefault(att[0]["gy"], []).append(st)
    dec = bench.get("decode", {})
    parts = ["# Kernel trace: cached decode steps (HIP-graph replay), BASELINE config 5\n\n"
             "Command (GPU box, repo root):\n\n```\n" + command + "\n```\n\n"
             "bench.py's decode measurement: prefill 128 tokens, then greedy steps, eager and "
             "then replayed from a captured `DecodeGraph`.  Steps are split after each step's "
             "last launch (the vocabulary argmax reduce) and grouped by batch (the decode "
             "attention kernel's grid y); the last 16 steps of each batch size (graph "
             "replays) are summarised.  Durations under the profiler.\n"]
    for b in sorted(by_batch):
        sts = by_batch[b][-16:]
        table, launches, busy, span = _step_table(sts)
        ref = dec.get(f"b{b}", {}).get("graph_decode_ms_per_step")
        parts.append(f"\n## batch {b}\n\nPer step: {launches:g} launches, {busy:.1f} us of "
                     f"kernel time, {span:.1f} us first start to last end"
                     + (f"; committed bench line: {ref * 1e3:.0f} us per step" if ref else "")
                     + ".\n\n" + table + "\n")
    (out_dir / "decode_graph_kernel_trace.md").write_text("".join(parts))
    return f"forwards {len(fwd)} x {mode} launches; decode batches {sorted(by_batch)}"


def load_json(path: Path) -> dict | None:
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return None


# ---------------------------------------------------------------------------

def build_model():
    """The default model (seed 2, bf16, HIP backends), the bs1x512 ids, and
    block 0's MoE input captured from one forward."""
    import torch

    from parrot import ModelConfig, Parrot, _abi
    _abi.load()  # fail loudly without the HIP library
    dev = torch.device("cuda:0")
    log("building model (seed 2)")
    torch.manual_seed(2)
    model = Parrot(ModelConfig(moe_backend="grouped_hip", depth_backend="hip",
                               collect_router_stats=False)).to(device=dev, dtype=torch.bfloat16)
    model.eval()
    ids = torch.randint(0, 32768, (1, TOKENS), generator=torch.Generator().manual_seed(2)).to(dev)

    captured = {}
    moe0 = model.blocks[0].moe
    originals = {name: getattr(moe0, name) for name in ("inference", "inference_then_mix")}

    def spying(name):
        def spy(x, **kw):
            captured.setdefault("x", x.detach().reshape(-1, x.shape[-1]).clone())
            return originals[name](x, **kw)
        return spy

    for name in originals:
        setattr(moe0, name, spying(name))
    with torch.no_grad():
        model(ids)
    for name in originals:
        delattr(moe0, name)
    if "x" not in captured:
        raise RuntimeError("block 0's MoE input was not captured")
    return model, ids, captured


def main():
    args = parse_args()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc))[:2000])
        return
    if args.summarize_steps:
        print(summarize_steps(args.summarize_steps))
        return
    if args.summarize_trace:
        print(json.dumps(summarize_trace(args.summarize_trace))[:2000])
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the MoE hot path has no multi-GPU implementation and "
              "every GPU box here has a single MI355X.", file=sys.stderr)
        sys.exit(2)
    if args.pmc_workload:
        pmc_workload()
        return

    import torch

    model, ids, captured = build_model()
    moe0 = model.blocks[0].moe
    if args.sweep_only:
        print(json.dumps({"sweep_E16": sweep_kernels(moe0, max(20, args.kernel_iters // 4))}),
              flush=True)
        return

    log("eager forward")
    with torch.no_grad():
        for _ in range(args.warmup):
            model(ids)
        torch.cuda.synchronize()
        eager = []
        for _ in range(max(3, args.steps // 4)):
            t0 = time.perf_counter()
            model(ids)
            torch.cuda.synchronize()
            eager.append(time.perf_counter() - t0)
    eager_ms = statistics.median(eager) * 1e3

    log("graph capture")
    static_ids = ids.clone()
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                model(static_ids)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_logits = model(static_ids).logits
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        reference_logits = model(ids).logits
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(static_logits, reference_logits):
            raise RuntimeError("graph replay differs from the eager forward")

        log(f"timed: {args.steps} graph replays")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    value = TOKENS * args.steps / elapsed
    del graph, static_logits, reference_logits

    kernels = {}
    roofline = None
    peaks = None
    if not args.skip_kernels:
        log("attained peaks")
        peaks = attained_peaks()
        ATTAINED.update(peaks)
        log("per-kernel timing")
        c4, _ = layer_kernels(moe0, captured["x"], args.kernel_iters, mark_roofline=True)
        kernels["C4_in_model_T512_E16"] = c4
        kernels.update(norm_kernels(model, args.kernel_iters))
        for name, tokens, skew in (("C2_T256_E32", 256, False), ("C3_T4096_E32_skew", 4096, True)):
            moe, x, bias = _layer_case(tokens, skew)
            kernels[name], _ = layer_kernels(moe, x, max(20, args.kernel_iters // 4), bias)
            del moe
        if not args.skip_sweep:
            log("token sweep")
            kernels["sweep_E16"] = sweep_kernels(moe0, max(20, args.kernel_iters // 4))
        # The forward's gate/up form at C4: grouping in-kernel, timed cold
        # (weights from HBM, as inside the forward); the warm loop beside it.
        gu, warm = c4["gate_up_grouping_cold"], c4["gate_up_grouping"]
        traffic = load_traffic()
        roofline = {"kernel": f"{TRAFFIC_KERNEL} (experts gate_up + SwiGLU, grouping the "
                              "top-2 ids in-kernel), C4 in-model shape T=512 E=16, cold: "
                              f"launches rotate over {gu['weight_copies']} copies of the "
                              "packed weights",
                    "bound": "hbm", "achieved": gu["gbps"], "peak": PEAK_HBM_GBPS,
                    "unit": "GB/s", "frac": gu["hbm_frac"], "traffic": traffic,
                    "algorithmic_bytes": gu["bytes"], "event_us": gu["us"],
                    "warm_event_us": warm["us"], "warm_frac": warm["hbm_frac"],
                    "attained_peak": peaks["copy_gbps"],
                    "frac_of_attained": round(gu["gbps"] / peaks["copy_gbps"], 4),
                    "traffic_source": str(PMC_FILE.relative_to(ROOT)) if traffic else None}
        trace = load_json(TRACE_FILE)
        if trace and trace.get("roofline_kernel") == TRAFFIC_KERNEL and trace.get("loop_mean_us"):
            # The committed kernel trace of this command: the same loop's mean
            # dispatch duration, and the kernel inside the graph-replayed forward.
            roofline["trace_source"] = str(TRACE_FILE.relative_to(ROOT))
            roofline["trace_loop_us"] = trace["loop_mean_us"]
            roofline["trace_loop_frac"] = round(
                gu["bytes"] / (trace["loop_mean_us"] * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)
            if trace.get("in_forward_mean_us"):
                roofline["in_forward_us"] = trace["in_forward_mean_us"]
                roofline["in_forward_frac"] = round(
                    gu["bytes"] / (trace["in_forward_mean_us"] * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)
        counters = load_json(PMC_FILE)
        if counters:
            kernels["counters_source"] = str(PMC_FILE.relative_to(ROOT))

    decode = None
    if not args.skip_decode:
        log("decode (config 5)")
        decode = decode_bench(model)

    result = {
        "metric": "tokens/sec Parrot bf16 fwd bs1x512 on 1 MI355X",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REFERENCE_TOK_S, 2),
        "baseline": "5,250 tokens/s: reference grouped_mps+metal on Apple M4 Pro, same workload "
                    "(README.md:42-44); no MI355X number is published",
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "Parrot default (16 layers, E=16 top-2 + shared, AttnRes, "
                               "vocab 32768) bf16 forward, batch 1 x 512, router stats off, "
                               "seed 2, HIP-graph replay",
                   "tokens": TOKENS, "moe_backend": "grouped_hip", "depth_backend": "hip"},
        "eager_ms_per_step": round(eager_ms, 3),
        "eager_tokens_per_s": round(TOKENS / (eager_ms / 1e3), 1),
        "roofline": roofline,
        "attained_peaks": peaks,
        "kernels": kernels,
        "decode": decode,
        "cpu_baseline": None,
    }
    if not args.skip_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(model, ids, args.cpu_seconds)
        result["cpu_baseline"]["moe_layers"] = cpu_layer_baselines(args.cpu_seconds)
    print(json.dumps(result), flush=True)


def _layer_case(tokens: int, skewed: bool, device="cuda", dtype=None):
    """MoE layer of BASELINE configs 2/3: E=32, weights N(0, 0.02), x N(0, 1)."""
    import torch
    dtype = torch.bfloat16 if dtype is None else dtype

    from parrot.model import ModelConfig, MoE
    cfg = ModelConfig(n_experts=32, moe_backend="grouped_hip", depth_backend="hip",
                      collect_router_stats=False)
    gen = torch.Generator().manual_seed(1)
    moe = MoE(cfg)
    with torch.no_grad():
        for p in moe.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    moe = moe.to(device=device, dtype=dtype).eval()
    x = torch.randn(tokens, cfg.dim, generator=torch.Generator().manual_seed(1)).to(
        device=device, dtype=dtype)
    bias = None
    if skewed:
        bias = torch.zeros(32)
        bias[0], bias[1] = 4.0, 2.0
    return moe, x, bias


if __name__ == "__main__":
    main()
