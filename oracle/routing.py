"""TEST INFRASTRUCTURE ONLY: routing / grouping oracle.

``top2``, ``positions``, ``group`` call the plain-C restatement in
oracle/route_group.c (built by ``make -C oracle``).  ``*_bruteforce`` are
independent pure-Python restatements for small inputs, used to pin the C
code.  Reference semantics (jkpdino/parrot-h200-worker):
  parrot/model.py:520-527 (softmax top-2, renormalised weights),
  parrot/model.py:547-551 (torch.where slot order),
  parrot/metal_moe.py:388-391 (capacity), :400-416 (exact overflow),
  parrot/kernels/moe_bf16.metal:104-118 (strict '>' selection).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "build" / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        p = ctypes.c_void_p
        lib.oracle_capacity.restype = ctypes.c_int32
        lib.oracle_capacity.argtypes = [ctypes.c_int64, ctypes.c_int32]
        lib.oracle_top2.restype = None
        lib.oracle_top2.argtypes = [p, p, ctypes.c_int64, ctypes.c_int32, p, p, p]
        lib.oracle_positions.restype = None
        lib.oracle_positions.argtypes = [p, ctypes.c_int64, ctypes.c_int32, p, p]
        lib.oracle_group.restype = None
        lib.oracle_group.argtypes = [p, p, p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                     p, p, p]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def capacity(tokens: int, experts: int) -> int:
    return int(_load().oracle_capacity(tokens, experts))


def top2(logits: np.ndarray, bias: np.ndarray | None = None, want_probs: bool = False):
    """(indices int64 [T, 2], weights fp32 [T, 2], probs fp32 [T, E] | None)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    tokens, experts = logits.shape
    if not 2 <= experts <= 64:
        raise ValueError("oracle supports 2..64 experts")
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    idx = np.empty((tokens, 2), dtype=np.int64)
    w = np.empty((tokens, 2), dtype=np.float32)
    probs = np.empty((tokens, experts), dtype=np.float32) if want_probs else None
    _load().oracle_top2(_ptr(logits), _ptr(bias), tokens, experts, _ptr(idx), _ptr(w),
                        _ptr(probs))
    return idx, w, probs


def positions(indices: np.ndarray, experts: int):
    """(positions int32 [2T], counts int32 [E]) with stable slot order."""
    flat = np.ascontiguousarray(indices.reshape(-1), dtype=np.int64)
    pos = np.empty(flat.shape[0], dtype=np.int32)
    counts = np.empty(experts, dtype=np.int32)
    _load().oracle_positions(_ptr(flat), flat.shape[0], experts, _ptr(pos), _ptr(counts))
    return pos, counts


def group(indices: np.ndarray, experts: int, cap: int | None = None):
    """Full grouping: dict with positions, counts, offsets, perm [E, C],
    overflow (valid prefix only) and capacity."""
    flat = np.ascontiguousarray(indices.reshape(-1), dtype=np.int64)
    tokens = flat.shape[0] // 2
    cap = capacity(tokens, experts) if cap is None else cap
    pos, counts = positions(flat, experts)
    perm = np.empty((experts, cap), dtype=np.int32)
    overflow = np.empty(max(flat.shape[0], 1), dtype=np.int32)
    offsets = np.empty(2 * experts + 2, dtype=np.int32)
    _load().oracle_group(_ptr(flat), _ptr(pos), _ptr(counts), flat.shape[0], experts, cap,
                         _ptr(perm), _ptr(overflow), _ptr(offsets))
    n_ovf = int(offsets[-1])
    return {"positions": pos, "counts": counts, "offsets": offsets, "perm": perm,
            "overflow": overflow[:n_ovf], "capacity": cap}


# ---- independent brute-force restatements (small inputs) -------------------

def top2_bruteforce(logits, bias=None):
    """Sort-based: order experts by (-logit, index), take the first two."""
    logits = np.asarray(logits, dtype=np.float32)
    if bias is not None:
        logits = logits + np.asarray(bias, dtype=np.float32)
    out = []
    for row in logits:
        order = sorted(range(len(row)), key=lambda e: (-float(row[e]), e))
        out.append(order[:2])
    return np.array(out, dtype=np.int64)


def group_bruteforce(indices, experts, cap):
    """Per expert, list its assignments in ascending a (torch.where order)."""
    flat = [int(v) for v in np.asarray(indices).reshape(-1)]
    perm = np.full((experts, cap), -1, dtype=np.int32)
    positions = np.zeros(len(flat), dtype=np.int32)
    overflow = []
    counts = np.zeros(experts, dtype=np.int32)
    for e in range(experts):
        mine = [a for a, v in enumerate(flat) if v == e]
        counts[e] = len(mine)
        for s, a in enumerate(mine):
            positions[a] = s
            if s < cap:
                perm[e, s] = a
            else:
                overflow.append(a)
    return {"positions": positions, "counts": counts, "perm": perm,
            "overflow": np.array(overflow, dtype=np.int32)}
