"""Pin the C routing/grouping oracle against independent restatements.

Checks: sort-based brute force for top-2, per-expert list brute force for
grouping, torch.where's row order (the reference's own ordering primitive,
parrot/model.py:548), the closed-form capacity values of the benchmark
configurations, and invariants (every assignment lands exactly once, the
overflow count is sum(max(0, count - C))).  A planted mistake (a '>=' tie
rule, a reversed slot order) is shown to fail these checks.
"""
import numpy as np
import pytest
import torch

from oracle import routing


@pytest.mark.parametrize("tokens,experts,expected", [
    (256, 32, 32),    # C2
    (4096, 32, 512),  # C3
    (512, 16, 128),   # C4
    (8, 16, 8), (1, 16, 8),  # C5 decode
    (64, 8, 32),      # tiny
    (0, 16, 8),
])
def test_capacity_closed_form(tokens, experts, expected):
    assert routing.capacity(tokens, experts) == expected


def test_capacity_formula_sweep():
    for tokens in range(0, 300, 7):
        for experts in (2, 3, 8, 16, 31, 32):
            assignments = 2 * tokens
            per_expert = -(-2 * assignments // experts)       # ceil(2A / E)
            c = max(8, -(-per_expert // 8) * 8)               # round up to 8
            assert routing.capacity(tokens, experts) == c


@pytest.mark.parametrize("experts", [2, 3, 8, 16, 32])
def test_top2_matches_sort_bruteforce(experts):
    rng = np.random.default_rng(experts)
    logits = rng.normal(size=(300, experts)).astype(np.float32)
    # plant exact ties in some rows
    logits[::7, 1] = logits[::7, 0]
    logits[::11, :] = 0.5
    idx, w, probs = routing.top2(logits, want_probs=True)
    np.testing.assert_array_equal(idx, routing.top2_bruteforce(logits))
    np.testing.assert_allclose(probs.sum(-1), 1.0, atol=1e-6)
    np.testing.assert_allclose(w.sum(-1), 1.0, atol=1e-6)
    assert (w[:, 0] >= w[:, 1]).all()
    # against torch softmax + topk where no ties exist
    clean = rng.normal(size=(200, experts)).astype(np.float32)
    tw, ti = torch.from_numpy(clean).softmax(-1).topk(2, -1)
    i2, w2, _ = routing.top2(clean)
    np.testing.assert_array_equal(i2, ti.numpy())
    np.testing.assert_allclose(w2, (tw / tw.sum(-1, keepdim=True)).numpy(), atol=1e-6)


def test_top2_bias_is_added_before_selection():
    logits = np.zeros((4, 8), dtype=np.float32)
    logits[:, 5] = 1.0
    bias = np.zeros(8, dtype=np.float32)
    bias[0], bias[1] = 4.0, 2.0
    idx, w, _ = routing.top2(logits, bias)
    assert (idx[:, 0] == 0).all() and (idx[:, 1] == 1).all()
    np.testing.assert_allclose(w[:, 0], 1 / (1 + np.exp(-2.0)), atol=1e-6)


def test_two_experts_select_both():
    rng = np.random.default_rng(0)
    idx, w, _ = routing.top2(rng.normal(size=(50, 2)).astype(np.float32))
    assert (np.sort(idx, -1) == [0, 1]).all()


def _random_indices(rng, tokens, experts, skew=None):
    idx = np.empty((tokens, 2), dtype=np.int64)
    for t in range(tokens):
        p = None if skew is None else skew
        idx[t] = rng.choice(experts, size=2, replace=False, p=p)
    return idx


@pytest.mark.parametrize("tokens,experts,skewed", [
    (1, 4, False), (7, 4, False), (64, 8, False), (200, 16, False), (300, 8, True), (257, 32, True)])
def test_group_matches_bruteforce(tokens, experts, skewed):
    rng = np.random.default_rng(tokens)
    skew = None
    if skewed:
        skew = np.full(experts, 0.05 / (experts - 2))
        skew[0], skew[1] = 0.7, 0.25
    idx = _random_indices(rng, tokens, experts, skew)
    cap = routing.capacity(tokens, experts)
    got = routing.group(idx, experts)
    ref = routing.group_bruteforce(idx, experts, cap)
    for key in ("positions", "counts", "perm", "overflow"):
        np.testing.assert_array_equal(got[key], ref[key], err_msg=key)
    # invariants
    seen = np.concatenate([got["perm"][got["perm"] >= 0], got["overflow"]])
    assert np.array_equal(np.sort(seen), np.arange(2 * tokens))
    assert int(got["offsets"][-1]) == int(np.maximum(got["counts"] - cap, 0).sum())
    np.testing.assert_array_equal(got["offsets"][:experts + 1],
                                  np.concatenate([[0], np.cumsum(got["counts"])]))


def test_group_order_is_torch_where_order():
    """Slots follow torch.where(indices == e) (parrot/model.py:548)."""
    rng = np.random.default_rng(5)
    idx = _random_indices(rng, 120, 8)
    got = routing.group(idx, 8, cap=1000)
    t_idx = torch.from_numpy(idx)
    for e in range(8):
        rows, slots = torch.where(t_idx == e)
        expect = (2 * rows + slots).numpy()
        np.testing.assert_array_equal(got["perm"][e, :len(expect)], expect)
        assert (got["perm"][e, len(expect):] == -1).all()


def test_all_tokens_one_expert_overflow():
    tokens, experts = 100, 8
    idx = np.stack([np.zeros(tokens), np.arange(tokens) % 7 + 1], 1).astype(np.int64)
    cap = routing.capacity(tokens, experts)  # 56
    got = routing.group(idx, experts)
    assert got["counts"][0] == tokens
    np.testing.assert_array_equal(got["overflow"][:tokens - cap], 2 * np.arange(cap, tokens))
    np.testing.assert_array_equal(got["perm"][0], 2 * np.arange(cap))


def test_round_robin_has_no_overflow():
    tokens, experts = 256, 16
    idx = np.stack([np.arange(tokens) % experts, (np.arange(tokens) + 1) % experts], 1)
    got = routing.group(idx.astype(np.int64), experts)
    assert int(got["offsets"][-1]) == 0 and got["overflow"].size == 0


def _top2_ge(row):
    """A plausible mistake: '>=' in the scan lets a later equal logit win."""
    first, second = (1, 0) if row[1] >= row[0] else (0, 1)
    for e in range(2, len(row)):
        if row[e] >= row[first]:
            first, second = e, first
        elif row[e] >= row[second]:
            second = e
    return [first, second]


def test_planted_mistakes_are_caught():
    """The checks above distinguish the oracle from plausible mistakes."""
    logits = np.array([[0.5, 0.5, 0.1], [0.3, 0.9, 0.9]], dtype=np.float32)
    brute = routing.top2_bruteforce(logits)
    np.testing.assert_array_equal(routing.top2(logits)[0], brute)
    assert [_top2_ge(r) for r in logits] != brute.tolist()
    # A reversed slot order disagrees with torch.where's order.
    idx = np.array([[0, 1], [0, 2], [0, 1]], dtype=np.int64)
    rows, slots = torch.where(torch.from_numpy(idx) == 0)
    got = routing.group(idx, 3, cap=8)
    np.testing.assert_array_equal(got["perm"][0, :3], (2 * rows + slots).numpy())
    assert list(got["perm"][0, :3][::-1]) != (2 * rows + slots).tolist()
