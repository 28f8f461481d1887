"""GPU check of the allocation-free grouped experts entry point
(parrot_grouped_experts_static_bf16): through the C ABI it gives the same
bits as parrot_grouped_experts_bf16 with a caller workspace, on two calls
in a row on the shared static array, the second with fewer tokens; it
allocates nothing through torch's allocator."""
import pytest
import torch

from moe_cases import inputs, moe_module, skew_bias

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _call_both(module, x, bias, addend):
    from parrot import _abi, hip_moe
    from parrot._abi import ptr
    lib = _abi.load()
    cfg = module.cfg
    tokens, dim = x.shape
    with torch.no_grad():
        routed = hip_moe.route(module, x, False, logit_bias=bias)
    g = routed.grouping
    gate_up, down, shared_gate_up, shared_down = hip_moe.pack_expert_weights(module)
    args = (tokens, dim, cfg.n_experts, cfg.expert_dim, cfg.shared_expert_dim, g.capacity,
            ptr(g.counts), ptr(g.offsets), ptr(g.perm), ptr(g.overflow), ptr(routed.weights),
            ptr(gate_up), ptr(down), ptr(shared_gate_up), ptr(shared_down), ptr(addend))
    stream = torch.cuda.current_stream().cuda_stream
    nbytes = lib.parrot_experts_workspace_bytes(tokens, dim, cfg.expert_dim,
                                                cfg.shared_expert_dim)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    want = torch.empty_like(x)
    _abi.check(lib.parrot_grouped_experts_bf16(ptr(x), *args, ptr(want), ptr(ws), nbytes,
                                               stream), "parrot_grouped_experts_bf16")
    got = torch.empty_like(x)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    _abi.check(lib.parrot_grouped_experts_static_bf16(ptr(x), *args, ptr(got), stream),
               "parrot_grouped_experts_static_bf16")
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    return got, want


def test_static_scratch_entry_matches_workspace_entry():
    module = moe_module(32, seed=1)
    # C3 (4096 tokens, skewed routing with overflow) fills the array exactly;
    # then C2 (256 tokens) with an addend reuses it.
    for tokens, bias, with_addend in [(4096, skew_bias(32), False), (256, None, True)]:
        _say(f"static-scratch grouped experts T={tokens} addend={with_addend}")
        x = inputs(tokens, seed=tokens)
        addend = inputs(tokens, seed=tokens + 1) if with_addend else None
        got, want = _call_both(module, x, bias, addend)
        assert torch.equal(got, want)


def test_static_scratch_entry_rejects_oversize_input():
    from parrot import _abi
    lib = _abi.load()
    status = lib.parrot_grouped_experts_static_bf16(
        None, 4097, 768, 32, 512, 256, 1032, *([None] * 11), None)
    assert status == -6
    assert b"static scratch" in lib.parrot_status_string(status)
