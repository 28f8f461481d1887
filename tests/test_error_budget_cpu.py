"""Where a bf16 forward's greedy argmax disagrees with the fp32 reference
(default model, seed 2, batch 1 x 512), attributed on the
CPU by switching the HIP forward's bf16 rounding points on and off in the
fp32 oracle (oracle/rounding_emulation.py).

Findings pinned here (the numbers also stand in the design notes):
  * with every rounding point on, ~3.5 % of token-layers pick a different
    top-2 than the fp32 model, and argmax agreement is ~94 %;
  * keeping the vocabulary logits in fp32 recovers a few tenths of a
    percent; keeping the AttnRes partial sums in fp32 recovers nothing;
  * forcing the fp32 model's own routing lifts agreement above 99 % and
    cuts the logits' max-abs error ~17x: top-2 flips at near-tied router
    logits carry nearly all of the disagreement.
"""
import numpy as np
import pytest
import torch

from oracle import parrot_fp32, rounding_emulation


def _agree(a, b):
    return (a.reshape(-1, a.shape[-1]).argmax(-1) == b.reshape(-1, b.shape[-1]).argmax(-1)) \
        .float().mean().item()


@pytest.fixture(scope="module")
def c4():
    from parrot import ModelConfig, Parrot
    torch.manual_seed(2)
    model = Parrot(ModelConfig(collect_router_stats=False)).to(torch.bfloat16)
    oracle = parrot_fp32.ParrotFP32(model.config, model.state_dict())
    del model
    ids = torch.randint(0, 32768, (1, 512), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        routes = []
        ref = rounding_emulation.forward(oracle, ids, act=False, stream=False, head_in=False,
                                         logit=False, capture=routes)
    return oracle, ids, ref, routes


def test_emulation_without_rounding_is_the_oracle(c4):
    oracle, ids, ref, _ = c4
    with torch.no_grad():
        assert torch.equal(ref, oracle.forward(ids))


def test_error_budget(c4):
    torch.set_num_threads(8)
    oracle, ids, ref, ref_routes = c4
    with torch.no_grad():
        routes = []
        all_bf16 = rounding_emulation.forward(oracle, ids, capture=routes)
        fp32_logits = rounding_emulation.forward(oracle, ids, logit=False)
        fp32_stream = rounding_emulation.forward(oracle, ids, logit=False, stream=False)
        forced = rounding_emulation.forward(oracle, ids, logit=False, force=ref_routes)
    flips = sum(int((np.sort(a, -1) != np.sort(b, -1)).any(-1).sum())
                for a, b in zip(routes, ref_routes))
    budget = {name: (_agree(v, ref), (v - ref).abs().max().item())
              for name, v in (("all bf16", all_bf16), ("fp32 logits", fp32_logits),
                              ("fp32 logits + stream", fp32_stream),
                              ("fp32 logits, fp32 routing", forced))}
    print(f"top-2 set flips: {flips} of {512 * 16}; {budget}")
    assert 0.01 < flips / (512 * 16) < 0.06
    assert budget["fp32 logits"][0] >= budget["all bf16"][0]
    assert budget["fp32 logits + stream"][0] <= budget["fp32 logits"][0] + 0.01
    assert budget["fp32 logits, fp32 routing"][0] >= 0.99
    assert budget["fp32 logits, fp32 routing"][1] * 10 < budget["fp32 logits"][1]


def test_bf16_noise_floor(c4):
    """The same bf16 rounding points with another accumulation order (every
    linear map accumulated in float64 before rounding) and the same routing
    move the C4 logits about as far as the bf16 rounding itself does: two
    bf16 forwards that differ only in fp32 reassociation agree on ~99 % of
    the greedy argmax positions, not 99.9 %.  Where a pre-rounding value sits
    within reassociation of a bf16 rounding boundary the two round
    differently, and sixteen layers of rounding carry that one-ulp
    difference to the size of the whole bf16 error.  So no bf16 forward
    (this build's, or the reference's own pytorch path in bf16) can be held
    to 99.9 % argmax agreement on all positions against another forward; the
    GPU test of the C4 forward compares the HIP forward against this floor
    (tests/test_gpu_model.py::test_default_forward_bf16_noise_floor)."""
    torch.set_num_threads(8)
    oracle, ids, ref, ref_routes = c4
    with torch.no_grad():
        emu = rounding_emulation.forward(oracle, ids, logit=False, force=ref_routes)
        emu64 = rounding_emulation.forward(oracle, ids, logit=False, force=ref_routes, acc64=True)
        exact64 = rounding_emulation.forward(oracle, ids, act=False, stream=False, head_in=False,
                                             logit=False, force=ref_routes, acc64=True)
    floor = _agree(emu, emu64)
    d_order = (emu - emu64).abs().mean().item()
    d_round = (emu - ref).abs().mean().item()
    print(f"bf16 vs bf16 (float64 accumulation): argmax {floor:.4f}, mean-abs {d_order:.2e}; "
          f"bf16 vs fp32 mean-abs {d_round:.2e}; fp32 vs fp32 (float64 accumulation) max-abs "
          f"{(exact64 - ref).abs().max().item():.2e}")
    # Without rounding the accumulation order changes the logits by ~1e-6 only.
    assert (exact64 - ref).abs().max().item() < 1e-4
    # With rounding it moves them by about as much as the rounding does.
    assert 0.5 * d_round < d_order < 1.5 * d_round
    assert 0.97 < floor < 0.999
