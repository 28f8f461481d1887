"""GPU parity of the full model on the HIP backend against the fp32 oracle.

Same seeded weights: the HIP model runs in bf16 on the GPU; the functional
fp32 oracle (oracle/parrot_fp32.py) runs on CPU with those bf16 weights
upcast.  Reported: logits max/mean abs error and argmax agreement.
"""
import numpy as np
import pytest
import torch

from conftest import tiny_model_config
from oracle import parrot_fp32

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _hip_model(cfg, seed):
    from parrot import Parrot
    torch.manual_seed(seed)
    return Parrot(cfg).to(device="cuda", dtype=torch.bfloat16).eval()


def _oracle(model):
    return parrot_fp32.ParrotFP32(model.config, model.state_dict())


def _compare(got, ref, min_agree):
    got = got.float().cpu().reshape(-1, got.shape[-1])
    ref = ref.float().cpu().reshape(-1, ref.shape[-1])
    agree = (got.argmax(-1) == ref.argmax(-1)).float().mean().item()
    d = (got - ref).abs()
    _say(f"  logits max-abs {d.max():.3e} mean-abs {d.mean():.3e} argmax agree {agree:.4f}")
    assert agree >= min_agree
    return agree


def test_tiny_forward():
    _say("tiny forward (grouped_hip + hip)")
    model = _hip_model(tiny_model_config(moe_backend="grouped_hip", depth_backend="hip",
                                         collect_router_stats=False), 0)
    ids = torch.randint(0, 32768, (2, 64), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        got = model(ids.cuda()).logits
        ref = _oracle(model).forward(ids)
    _compare(got, ref, 0.95)


def test_tiny_router_stats():
    _say("tiny forward with router stats")
    model = _hip_model(tiny_model_config(moe_backend="grouped_hip", depth_backend="hip"), 0)
    ids = torch.randint(0, 32768, (1, 64), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        out = model(ids.cuda())
    util = out.expert_utilization.cpu()
    torch.testing.assert_close(util.sum(-1), torch.ones(4))
    assert torch.isfinite(out.aux_loss).item()


def test_default_forward_512():
    """default model (E=16), seed 2, batch 1 x 512.

    The HIP path must agree with the fp32 oracle at least as well as the
    plain PyTorch bf16 execution of the same model and weights (the
    reference's pytorch backend in bf16), which bounds what bf16 can reach
    on this random-init model: ~14% of positions have an fp32 top-1/top-2
    logit gap below 0.02, while 16 layers of bf16 activations move the
    logits by ~0.013 on average."""
    from parrot import ModelConfig, Parrot
    _say("default forward 1x512 (seed 2)")
    model = _hip_model(ModelConfig(moe_backend="grouped_hip", depth_backend="hip",
                                   collect_router_stats=False), 2)
    control = Parrot(ModelConfig(collect_router_stats=False))
    control.load_state_dict(model.state_dict())
    control = control.to(device="cuda", dtype=torch.bfloat16).eval()
    ids = torch.randint(0, 32768, (1, 512), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        got = model(ids.cuda()).logits
        base = control(ids.cuda()).logits
    ref = _oracle(model).forward(ids)
    agree = _compare(got, ref, 0.9)
    control_agree = _compare(base, ref, 0.9)
    _say(f"  argmax agreement: HIP {agree:.4f}, PyTorch bf16 control {control_agree:.4f}")
    assert agree >= control_agree - 0.01
    d = (got.float().cpu() - ref.float()).abs()
    assert d.mean() < 0.02


def test_prefill_and_decode():
    """BASELINE config 5 shape at reduced length: prefill then greedy decode."""
    from parrot import ModelConfig
    _say("prefill 128 + 4 decode steps, batch 2")
    model = _hip_model(ModelConfig(moe_backend="grouped_hip", depth_backend="hip",
                                   collect_router_stats=False), 3)
    oracle = _oracle(model)
    prompt = torch.randint(0, 32768, (2, 128), generator=torch.Generator().manual_seed(3))
    logits, state = model.prefill(prompt.cuda())
    ref_logits, ref_state = oracle.prefill(prompt)
    _compare(logits, ref_logits, 0.5)
    for step in range(4):
        nxt = ref_logits[:, -1].argmax(-1, keepdim=True)  # feed identical tokens
        logits, state = model.decode_step(nxt.cuda(), state)
        ref_logits = oracle.decode_step(nxt, ref_state)
        _compare(logits, ref_logits, 0.5)
    assert state.position == 132


def test_graph_replay_matches_eager():
    """The forward captured in a HIP graph replays identically (several
    replays, with eager work and synchronisation in between)."""
    from parrot import ModelConfig
    _say("graph capture replay")
    model = _hip_model(ModelConfig(n_layers=4, moe_backend="grouped_hip", depth_backend="hip",
                                   collect_router_stats=False), 5)
    ids = torch.randint(0, 32768, (1, 512), generator=torch.Generator().manual_seed(5)).cuda()
    static_ids = ids.clone()
    with torch.no_grad():
        eager = model(ids).logits.clone()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(2):
                model(static_ids)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out = model(static_ids).logits
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager)
            model(ids)  # eager work between replays
            torch.cuda.synchronize()


def test_routing_in_depth_mix_matches_separate_launches(monkeypatch):
    """The forward and prefill whose MoE input depth mixes also route (and
    whose gate/up launches group in-kernel) equal, bit for bit, the same
    model with separate route and grouping launches."""
    from parrot import ModelConfig
    from parrot.model import MoE
    _say("routing in the depth mix vs separate launches")
    model = _hip_model(ModelConfig(n_layers=4, moe_backend="grouped_hip", depth_backend="hip",
                                   collect_router_stats=False), 6)
    ids = torch.randint(0, 32768, (2, 200), generator=torch.Generator().manual_seed(6)).cuda()
    with torch.no_grad():
        assert model.blocks[0].moe.routes_in_depth_mix(
            torch.empty(400, 768, dtype=torch.bfloat16, device="cuda"))
        fused = model(ids).logits
        fused_prefill, _ = model.prefill(ids)
        monkeypatch.setattr(MoE, "routes_in_depth_mix", lambda self, x: False)
        separate = model(ids).logits
        separate_prefill, _ = model.prefill(ids)
    assert torch.equal(fused, separate)
    assert torch.equal(fused_prefill, separate_prefill)
