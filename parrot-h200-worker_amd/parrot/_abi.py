"""ctypes binding of ``libparrot_hip.so`` (C ABI in ``include/parrot_hip.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime
(``libamdhip64.so.7``) that PyTorch-ROCm already mapped; both then share
devices, streams and the caching allocator's memory.  There is no fallback:
if the library is missing, every HIP entry point raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (maps PyTorch's HIP runtime before the library)

LIBRARY = Path(__file__).resolve().parent / "_lib" / "libparrot_hip.so"
ABI_VERSION = 14

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/parrot_hip.h
SIGNATURES: dict[str, tuple] = {
    "parrot_abi_version": (ctypes.c_int, []),
    "parrot_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "parrot_capacity": (_i32, [_i64, _i32]),
    "parrot_rms_norm_bf16": (ctypes.c_int, [_p, _p, _p, _i64, _i32, _f32, _p]),
    "parrot_depth_mix_bf16": (
        ctypes.c_int, [_p, _i32, _p, _p, _f32, _p, _f32, _i64, _i32, _p, _p, _p]),
    "parrot_embed_depth_mix_bf16": (
        ctypes.c_int,
        [_p, _i64, _p, _i64, _i32, _p, _p, _f32, _p, _f32, _p, _p, _p, _i32, _p]),
    "parrot_rope_qkv_bf16": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i32, _i32, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p]),
    "parrot_decode_attention_bf16": (
        ctypes.c_int,
        [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p]),
    "parrot_decode_attention_heads_bf16": (
        ctypes.c_int,
        [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p, _i32, _p, _p]),
    "parrot_decode_attention_heads_check": (
        ctypes.c_int, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "parrot_decode_moe_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "parrot_vocab_argmax_workspace_bytes": (_sz, [_i64, _i32]),
    "parrot_causal_attention_bf16": (
        ctypes.c_int, [_p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p]),
    "parrot_causal_attention_frag_bf16": (
        ctypes.c_int, [_p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p]),
    "parrot_proj_rope_qkv_frag_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _p, _p, _p, _i32, _p, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p,
         _p]),
    "parrot_proj_frag_bf16": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _i32, _i32, _i32, _p, _p]),
    "parrot_experts_combine_depth_mix_bf16": (
        ctypes.c_int,
        [_i64, _i32, _i32, _i32, _p, _p, _p, _sz, _p, _i32, _p, _p, _f32, _p, _f32, _p, _p, _p]),
    "parrot_proj_kv_frag_bf16": (
        ctypes.c_int, [_p, _i64, _i32, _i32, _i64, _p, _i32, _i32, _p, _p, _p]),
    "parrot_proj_bf16": (ctypes.c_int, [_p, _i64, _i32, _i64, _p, _i32, _p, _i64, _p, _i64, _p]),
    "parrot_proj_transposed_bf16": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _i32, _i32, _p, _p]),
    "parrot_proj_rope_qkv_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _p, _p, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p]),
    "parrot_vocab_argmax_bf16": (ctypes.c_int, [_p, _i64, _i32, _p, _i32, _p, _p, _p, _sz, _p]),
    "parrot_causal_attention_frag_out_bf16": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i32, _i32, _i32,
                                                              _i32, _i32, _f32, _p, _i32, _p, _p]),
    "parrot_depth_mix_route_pending_bf16": (ctypes.c_int, [_p, _i32, _p, _p, _f32, _p, _f32, _i64,
                                                            _i32, _p, _p, _p, _i32, _p, _p, _p,
                                                            _i32, _p, _p, _p]),
    "parrot_decode_moe_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_depth_mix_decode_moe_bf16": (
        ctypes.c_int,
        [_p, _i32, _p, _p, _f32, _p, _f32, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p,
         _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_depth_mix_decode_moe_pending_bf16": (
        ctypes.c_int,
        [_p, _i32, _p, _p, _f32, _p, _f32, _p, _i32, _p, _p, _i64, _i32, _i32, _i32, _i32, _p,
         _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_decode_attention_latent_f32": (
        ctypes.c_int, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _f32, _p, _p]),
    "parrot_route_workspace_bytes": (_sz, [_i64, _i32]),
    "parrot_route_bf16": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_route_from_logits_f32": (
        ctypes.c_int, [_p, _p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_group_indices": (
        ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_experts_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32]),
    "parrot_experts_gate_up_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_experts_down_bf16": (
        ctypes.c_int,
        [_i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_experts_combine_bf16": (
        ctypes.c_int, [_i64, _i32, _i32, _i32, _p, _p, _p, _sz, _p]),
    "parrot_depth_mix_route_bf16": (
        ctypes.c_int,
        [_p, _i32, _p, _p, _f32, _p, _f32, _i64, _i32, _p, _p, _p, _p, _i32, _p, _p, _p]),
    "parrot_experts_group_in_kernel": (ctypes.c_int, [_i64, _i32, _i32, _i32, _i32]),
    "parrot_decode_qkv_bf16": (
        ctypes.c_int,
        [_p, _p, _i32, _p, _p, _f32, _p, _f32, _i32, _i32, _p, _i32, _i32, _i32, _p, _p, _i32,
         _p, _p, _p, _p, _p]),
    "parrot_decode_qkv_embed_bf16": (
        ctypes.c_int,
        [_p, _p, _i32, _p, _p, _p, _f32, _p, _f32, _i32, _i32, _p, _i32, _i32, _i32, _p, _p,
         _i32, _p, _p, _p, _p, _p]),
    "parrot_mla_decode_in_bf16": (
        ctypes.c_int,
        [_p, _p, _i32, _p, _p, _f32, _p, _f32, _i32, _i32, _p, _i32, _p, _i32, _p, _p, _p]),
    "parrot_mla_decode_out_bf16": (ctypes.c_int, [_p, _i32, _i32, _p, _i32, _p, _p, _p]),
    "parrot_decode_linear_bf16": (ctypes.c_int, [_p, _i32, _i32, _p, _i32, _p, _p, _p]),
    "parrot_experts_gate_up_grouping_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_experts_gate_up_grouping_blocks_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_experts_down_sorted_bf16": (
        ctypes.c_int,
        [_i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "parrot_grouped_experts_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
         _p, _sz, _p]),
    "parrot_route_top2_bf16": (ctypes.c_int, [_p, _p, _p, _i64, _i32, _i32, _p, _p, _p]),
    "parrot_route_top2_blocks_bf16": (
        ctypes.c_int, [_p, _p, _p, _i64, _i32, _i32, _p, _p, _p, _p]),
    "parrot_peak_mfma_bf16": (ctypes.c_int, [_i32, _i64, _i32, _p, _p, _p]),
    "parrot_peak_copy": (ctypes.c_int, [_p, _p, _i64, _i64, _p]),
    "parrot_grouped_experts_static_bf16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
         _p]),
}

STATIC_SCRATCH_BYTES = 30 << 20  # PARROT_STATIC_SCRATCH_BYTES

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load and type the library once; raise if it is absent or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        raise RuntimeError(
            f"HIP extension not built: {LIBRARY} is missing "
            "(run __graft_entry__.build() or `python -m parrot._build`)")
    lib = ctypes.CDLL(str(LIBRARY))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.parrot_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libparrot_hip ABI {version}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        message = load().parrot_status_string(status).decode()
        raise RuntimeError(f"{what} failed with status {status}: {message}")


def ptr(tensor) -> int | None:
    """Device address of a tensor (None passes NULL)."""
    return None if tensor is None else tensor.data_ptr()
