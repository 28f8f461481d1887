"""GPU parity: routing and grouping are bit-exact with the C oracle.

Contract: given identical fp32 router logits, the top-2 indices, every
per-expert slot permutation and the overflow assignment are bit-exact
(route weights / probabilities within 1e-6).  The HIP projection's own
logits are checked against fp32 and then run through the oracle's top-2.
"""
import numpy as np
import pytest
import torch

from moe_cases import inputs, moe_module, skew_bias
from oracle import routing

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _assert_grouping_equal(g, ref):
    np.testing.assert_array_equal(g.positions.cpu().numpy(), ref["positions"])
    np.testing.assert_array_equal(g.counts.cpu().numpy(), ref["counts"])
    np.testing.assert_array_equal(g.offsets.cpu().numpy(), ref["offsets"])
    np.testing.assert_array_equal(g.perm.cpu().numpy(), ref["perm"])
    n = int(ref["offsets"][-1])
    np.testing.assert_array_equal(g.overflow.cpu().numpy()[:n], ref["overflow"])


CASES = [(256, 32, False), (4096, 32, True), (512, 16, False), (1, 16, False), (3, 16, False),
         (8, 16, False), (64, 8, False), (1000, 2, False), (130, 3, False), (777, 32, True),
         (16384, 16, False)]


@pytest.mark.parametrize("tokens,experts,skewed", CASES)
def test_route_from_logits_bit_exact(tokens, experts, skewed):
    from parrot import hip_moe
    _say(f"route_from_logits T={tokens} E={experts} skew={skewed}")
    rng = np.random.default_rng(tokens * 31 + experts)
    logits = (rng.normal(size=(tokens, experts)) * 0.55).astype(np.float32)
    logits[::13, 1] = logits[::13, 0]  # exact ties
    bias = skew_bias(experts).numpy() if skewed else None
    res = hip_moe.route_from_logits(torch.from_numpy(logits).cuda(),
                                    None if bias is None else torch.from_numpy(bias),
                                    collect_stats=True)
    idx, w, probs = routing.top2(logits, bias, want_probs=True)
    np.testing.assert_array_equal(res.indices.cpu().numpy(), idx)
    np.testing.assert_allclose(res.weights.cpu().numpy(), w, atol=1e-6, rtol=0)
    np.testing.assert_allclose(res.probabilities.cpu().numpy(), probs, atol=1e-6, rtol=0)
    ref = routing.group(idx, experts)
    assert res.grouping.capacity == ref["capacity"]
    _assert_grouping_equal(res.grouping, ref)
    if skewed:
        _say(f"  overflow assignments: {int(ref['offsets'][-1])} of {2 * tokens}")


@pytest.mark.parametrize("tokens,experts,skewed", [(256, 32, False), (4096, 32, True),
                                                   (512, 16, False), (5, 16, False),
                                                   (16421, 16, False), (20000, 32, True),
                                                   (32800, 16, False), (40000, 32, True)])
def test_route_projection(tokens, experts, skewed):
    """HIP logits ~ fp32 logits; HIP top-2 == oracle top-2 of the HIP logits."""
    from parrot import hip_moe
    _say(f"route projection T={tokens} E={experts} skew={skewed}")
    module = moe_module(experts, seed=1)
    x = inputs(tokens, seed=1)
    bias = skew_bias(experts) if skewed else None
    with torch.no_grad():
        res = hip_moe.route(module, x, collect_stats=True, logit_bias=bias, return_logits=True)
    got_logits = res.logits.cpu().numpy()
    ref_logits = (x.float().cpu() @ module.router.weight.detach().float().cpu().T).numpy()
    if bias is not None:
        ref_logits = ref_logits + bias.numpy()
    assert np.abs(got_logits - ref_logits).max() < 1e-4
    idx, w, _ = routing.top2(got_logits)
    np.testing.assert_array_equal(res.indices.cpu().numpy(), idx)
    np.testing.assert_allclose(res.weights.cpu().numpy(), w, atol=1e-6)
    _assert_grouping_equal(res.grouping, routing.group(idx, experts))
    # With the fp32 oracle's own logits, routing agrees except at near-ties.
    ref_idx, _, _ = routing.top2(ref_logits)
    mismatch = (ref_idx != idx).any(-1).mean()
    assert mismatch <= 0.002, mismatch


def test_group_indices_adversarial():
    from parrot import hip_moe
    cases = {
        "one_expert": np.stack([np.zeros(3000), np.arange(3000) % 15 + 1], 1),
        "round_robin": np.stack([np.arange(512) % 16, (np.arange(512) + 1) % 16], 1),
        "two_experts": np.stack([np.zeros(700), np.ones(700)], 1),
        # long enough for the two-level histogram scan (> 256 route blocks)
        "long_skewed": np.stack([np.zeros(40001), np.arange(40001) % 7 + 1], 1),
        "long_uniform": np.stack([np.arange(9000) % 16, (np.arange(9000) * 5 + 3) % 16], 1),
    }
    for name, idx in cases.items():
        _say(f"group_indices {name}")
        idx = idx.astype(np.int64)
        g = hip_moe.group_indices(torch.from_numpy(idx).cuda(), 16)
        _assert_grouping_equal(g, routing.group(idx, 16))


def test_routing_is_deterministic():
    from parrot import hip_moe
    _say("routing determinism")
    module = moe_module(32, seed=1)
    x = inputs(4096, seed=3)
    with torch.no_grad():
        a = hip_moe.route(module, x, False, logit_bias=skew_bias(32))
        b = hip_moe.route(module, x, False, logit_bias=skew_bias(32))
    for name in ("positions", "counts", "offsets", "perm"):
        assert torch.equal(getattr(a.grouping, name), getattr(b.grouping, name)), name
    n = int(a.grouping.offsets[-1])  # valid prefix of the overflow list
    assert torch.equal(a.grouping.overflow[:n], b.grouping.overflow[:n])
    assert torch.equal(a.indices, b.indices) and torch.equal(a.weights, b.weights)


@pytest.mark.parametrize("experts", [16, 32])
def test_wide_route_matches_split_k_chunks(experts):
    """From 32768 tokens the router runs one 64-token kernel whose logits
    keep four k-step chains (st % 4) summed in route_kernel's order, so a
    token's logits, top-2 and weights are the same bits as when its rows are
    routed in chunks below 32768 tokens (split-K kernel): routing does not
    depend on the batch size."""
    from parrot import hip_moe
    _say(f"wide route vs split-K chunks T=32800 E={experts}")
    module = moe_module(experts, seed=7)
    x = inputs(32800, seed=7)
    with torch.no_grad():
        wide = hip_moe.route(module, x, collect_stats=False, return_logits=True)
        parts = [hip_moe.route(module, x[lo:lo + 16400], collect_stats=False, return_logits=True)
                 for lo in (0, 16400)]
    assert torch.equal(wide.logits, torch.cat([p.logits for p in parts]))
    assert torch.equal(wide.indices, torch.cat([p.indices for p in parts]))
    assert torch.equal(wide.weights, torch.cat([p.weights for p in parts]))


@pytest.mark.parametrize("tokens,experts,skewed", [(256, 32, False), (4096, 32, True),
                                                   (513, 16, False), (32800, 16, False)])
def test_route_top2_matches_route(tokens, experts, skewed):
    """The top-2-only entry gives route()'s weights and indices bit for bit."""
    from parrot import hip_moe
    _say(f"route_top2 T={tokens} E={experts} skew={skewed}")
    module = moe_module(experts, seed=2)
    x = inputs(tokens, seed=2)
    bias = skew_bias(experts) if skewed else None
    with torch.no_grad():
        full = hip_moe.route(module, x, collect_stats=False, logit_bias=bias)
        top2 = hip_moe.route_top2(module, x, logit_bias=bias)
    assert top2.grouping is None
    assert torch.equal(full.indices, top2.indices)
    assert torch.equal(full.weights, top2.weights)
    if tokens >= 32768:
        return  # the block table is written below the wide router's sizes
    with torch.no_grad():
        tab = hip_moe.route_top2(module, x, logit_bias=bias, blocks=True)
    assert torch.equal(full.indices, tab.indices) and torch.equal(full.weights, tab.weights)
    # The table from the indices: per 16 tokens the 32 ids in assignment
    # order (255 for padding tokens), then the count of each expert.
    ids = full.indices.reshape(-1).cpu().numpy()
    n_blocks = (tokens + 15) // 16
    padded = np.full(n_blocks * 32, 255, dtype=np.int64)
    padded[:ids.size] = ids
    rows = padded.reshape(n_blocks, 32)
    counts = np.stack([(rows == e).sum(axis=1) for e in range(32)], axis=1)
    want = np.concatenate([rows, counts], axis=1).astype(np.uint8)
    assert np.array_equal(tab.blocks.cpu().numpy(), want)


def test_route_unpacks_as_metal_route():
    """route() unpacks as metal_route's 5-tuple (parrot/metal_moe.py:58-81),
    so the reference's call site (parrot/model.py:515-519) reads it as is."""
    from parrot import hip_moe
    _say("route unpacks as metal_route")
    module = moe_module(16, seed=1)
    x = inputs(300, seed=2)
    with torch.no_grad():
        res = hip_moe.route(module, x, collect_stats=True)
        probabilities, weights, indices, positions, counts = res
        plain = hip_moe.route(module, x, collect_stats=False)
    assert probabilities is res.probabilities and probabilities.shape == (300, 16)
    assert weights is res.weights and indices is res.indices
    assert positions is res.grouping.positions and counts is res.grouping.counts
    assert int(counts.sum()) == 600 and tuple(plain)[0] is None
